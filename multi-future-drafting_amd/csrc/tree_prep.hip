// Inputs of tree-GDN verification for gfx950: the short causal convolution of every tree node over its
// window of ancestors, SiLU, and the q / k normalisation (inference/hf/tree_gdn_kernel.py:29-56 _tree_prep,
// :135-150 tree_prep), and the windows themselves (inference/hf/qwen35_tree.py:39-52 TreeContext.conv_index).
//
// Window of node i (oldest first): the conv_kernel most recent inputs on its root path, i.e. i, its parent,
// grandparent, ..., and, above the root, the cached conv state from its most recent column backwards. An
// entry is an index into [conv state (KC columns) ; the request's nodes].
//
// tree_prep, channel c of node i (channels in the order q heads, k heads, v heads, D = 128 each):
//   acc = sum_t w[c][t] * win_t(c)  (fp32; the product of two bf16 values is exact, so one rounding per tap)
//   y   = bf16(acc * sigmoid(acc))  (rounded as the model's own path rounds the activation)
//   q, k: y * rsqrt(sum_{c in head} y^2 + 1e-6), q also times scale;  stored as bf16.
// One wave per (block of 4 nodes, 512 channels = 4 heads); lane l owns 8 consecutive channels, so its
// weight and conv-state rows are one contiguous 8 KC-element run (loaded once for the 4 nodes), a tap's x
// read is a 16-byte segment, and a head's 16 lanes form one DPP row for the sum of squares. The windows
// (scalar loads) and x rows of 2 nodes are issued before any is used.
#include "mfd_common.h"

namespace {

constexpr int D = 128;
constexpr int KC_MAX = 8;

struct PrepArgs {
  const uint16_t* x;   // [N, CD] bf16, row stride x_st
  int64_t x_st;
  const uint16_t* cs;  // conv state [R][CD][KC] bf16, request stride cs_rst
  int64_t cs_rst;
  const int32_t* cidx; // [N, KC] request-local window indices
  const uint16_t* w;   // [CD, KC] bf16
  const int32_t* cu;   // [R + 1] node offsets or null (one request)
  int R, N, HK, H, hg_blocks;
  float scale;
  uint16_t* q;         // [N, HK, D]
  uint16_t* k;         // [N, HK, D]
  uint16_t* v;         // [N, H, D]
  int32_t* err;        // optional: MFD_DEVERR_BAD_WINDOW when a window index is out of range
};

// request of node i: the last r with cu[r] <= i (wave-uniform binary search)
__device__ __forceinline__ int request_of(const int32_t* cu, int R, int i) {
  int lo = 0, hi = R - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= i) lo = mid; else hi = mid - 1;
  }
  return lo;
}

template <int N>
__device__ __forceinline__ float row_ror_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}
// sum over the 64 lanes (wave-uniform result)
__device__ __forceinline__ float wave_sum(float v) {
  v += row_ror_f<1>(v);
  v += row_ror_f<2>(v);
  v += row_ror_f<4>(v);
  v += row_ror_f<8>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

typedef uint32_t u32x4p __attribute__((ext_vector_type(4)));

constexpr int NB = 4;   // nodes per workgroup
constexpr int NU = 2;   // nodes whose loads are issued together
constexpr int CPL = 8;  // channels per lane: 16 lanes (one DPP row) cover one head

template <int N>
__device__ __forceinline__ float row_ror_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}

template <int KC>
__global__ __launch_bounds__(256) void tree_prep_kernel(PrepArgs a) {
  typedef const __attribute__((address_space(4))) int32_t* const_i32p;  // scalar loads of uniform indices
  const int lane = threadIdx.x & 63;
  const int nblk = blockIdx.x / a.hg_blocks;
  const int CD = (2 * a.HK + a.H) * D;
  const int c0 = ((blockIdx.x % a.hg_blocks) * 4 + (threadIdx.x >> 6)) * (64 * CPL) + lane * CPL;
  if (__builtin_amdgcn_readfirstlane(c0 - lane * CPL) >= CD) return;  // a wave past the last channel
  const bool live = c0 < CD;
  const int cl = live ? c0 : 0;  // lanes past the last channel compute on channel 0 and store nothing
  const int head = cl / D;
  const bool is_q = head < a.HK, is_qk = head < 2 * a.HK;
  const int i0 = nblk * NB, i1 = min(i0 + NB, a.N);
  // request offsets held one per lane (more than 63 requests: binary search)
  const int cu_l = a.cu ? (lane <= a.R ? a.cu[lane] : 0x7FFFFFFF) : (lane == 0 ? 0 : a.N);
  auto request_of_node = [&](int i) -> int {
    if (a.cu && a.R > 63) return request_of(a.cu, a.R, i);
    const uint64_t m = __builtin_amdgcn_ballot_w64(lane <= (a.cu ? a.R : 1) && cu_l <= i);
    return (int)__builtin_popcountll(m) - 1;
  };
  auto offset_of = [&](int r) -> int {
    if (!a.cu) return r == 0 ? 0 : a.N;
    if (a.R > 63) return a.cu[r];
    return __builtin_amdgcn_readlane(cu_l, r);
  };
  // the lane's CPL weight rows (CPL * KC contiguous elements) and conv-state rows of the current request
  // (element c * KC + t of a run is channel c, window position t); the weights held as bf16 pairs of
  // positions (2p, 2p + 1) per channel, the second weight 0 past the last position (odd KC)
  constexpr int KP = (KC + 1) / 2;
  uint32_t wpair[CPL][KP];
  u16x8 sraw[KC];
  {
    const u16x8* wp = reinterpret_cast<const u16x8*>(a.w + (int64_t)cl * KC);
    u16x8 wraw[KC];
#pragma unroll
    for (int e = 0; e < KC; ++e) wraw[e] = wp[e];
#pragma unroll
    for (int c = 0; c < CPL; ++c)
#pragma unroll
      for (int p = 0; p < KP; ++p) {
        const int j = c * KC + 2 * p;
        const uint32_t hi = 2 * p + 1 < KC ? (uint32_t)wraw[(j + 1) / 8][(j + 1) % 8] : 0u;
        wpair[c][p] = (uint32_t)wraw[j / 8][j % 8] | (hi << 16);
      }
  }
  int r_cur = -1;
  for (int ib = i0; ib < i1; ib += NU) {
    int rq[NU], base[NU], nloc[NU];
    int32_t ix[NU][KC];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int node = min(ib + u, i1 - 1);
      rq[u] = request_of_node(node);
      base[u] = offset_of(rq[u]);
      nloc[u] = offset_of(rq[u] + 1) - base[u];
#pragma unroll
      for (int t = 0; t < KC; ++t) ix[u][t] = ((const_i32p)a.cidx)[(int64_t)node * KC + t];
    }
    // every x row segment of the NU windows, loaded before any is used
    u16x8 xr[NU][KC];
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int t = 0; t < KC; ++t) {
        const int idx = ix[u][t];
        // a row outside the request's nodes is not loaded: the sum below reads xr only for the rows loaded here
        if (idx >= KC && idx < KC + nloc[u])
          xr[u][t] = *reinterpret_cast<const u16x8*>(a.x + (int64_t)(base[u] + idx - KC) * a.x_st + cl);
      }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int node = ib + u;
      if (node >= i1) break;
      if (rq[u] != r_cur) {  // conv state of this node's request
        r_cur = rq[u];
        const u16x8* sp = reinterpret_cast<const u16x8*>(a.cs + (int64_t)r_cur * a.cs_rst + (int64_t)cl * KC);
#pragma unroll
        for (int e = 0; e < KC; ++e) sraw[e] = sp[e];
      }
      // the window's KC rows of the lane's 8 channels as bf16 (two channels a word); a position outside
      // [conv state ; request's nodes] contributes 0 and is flagged
      u32x4p row[KC];
#pragma unroll
      for (int t = 0; t < KC; ++t) {
        const int idx = ix[u][t];
        if (idx < 0 || idx >= KC + nloc[u]) {
          if (lane == 0 && a.err) atomicOr(a.err, MFD_DEVERR_BAD_WINDOW);
          row[t] = (u32x4p){0u, 0u, 0u, 0u};
        } else if (idx < KC) {
          // column idx of the cached state, selected from registers (idx is wave-uniform)
          u32x4p r = {0u, 0u, 0u, 0u};
#pragma unroll
          for (int e = 0; e < KC; ++e)
            if (e == idx) {
#pragma unroll
              for (int k = 0; k < CPL / 2; ++k) {
                const int j0 = 2 * k * KC + e, j1 = (2 * k + 1) * KC + e;
                r[k] = (uint32_t)sraw[j0 / 8][j0 % 8] | ((uint32_t)sraw[j1 / 8][j1 % 8] << 16);
              }
            }
          row[t] = r;
        } else {
          row[t] = __builtin_bit_cast(u32x4p, xr[u][t]);
        }
      }
      // acc = sum over t of w[c][t] * row_t[c] in fp32 (each bf16 product exact), two positions per
      // v_dot2_f32_bf16: v_perm pairs channel c of rows 2p and 2p + 1
      float acc[CPL];
#pragma unroll
      for (int c = 0; c < CPL; ++c) acc[c] = 0.f;
#pragma unroll
      for (int p = 0; p < KP; ++p)
#pragma unroll
        for (int k = 0; k < CPL / 2; ++k) {
          const uint32_t r0 = row[2 * p][k], r1 = 2 * p + 1 < KC ? row[2 * p + 1][k] : 0u;
          const uint32_t lo = __builtin_amdgcn_perm(r1, r0, 0x05040100u);  // channel 2k of both rows
          const uint32_t hi = __builtin_amdgcn_perm(r1, r0, 0x07060302u);  // channel 2k + 1
          acc[2 * k] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wpair[2 * k][p]),
                                                       __builtin_bit_cast(bf16x2, lo), acc[2 * k], false);
          acc[2 * k + 1] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wpair[2 * k + 1][p]),
                                                           __builtin_bit_cast(bf16x2, hi), acc[2 * k + 1], false);
        }
      // SiLU rounded to bf16, the head's sum of squares over its 16 lanes (one DPP row)
      float y[CPL];
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; c += 2) {  // two channels rounded to bf16 by one packed conversion
        const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(
            (f32x2){acc[c] * __builtin_amdgcn_rcpf(1.f + __expf(-acc[c])),
                    acc[c + 1] * __builtin_amdgcn_rcpf(1.f + __expf(-acc[c + 1]))}, bf16x2));
        y[c] = __uint_as_float(p << 16);
        y[c + 1] = __uint_as_float(p & 0xFFFF0000u);
        ss = __builtin_fmaf(y[c], y[c], ss);
        ss = __builtin_fmaf(y[c + 1], y[c + 1], ss);
      }
      ss = row_ror_add<1>(ss);
      ss = row_ror_add<2>(ss);
      ss = row_ror_add<4>(ss);
      ss = row_ror_add<8>(ss);
      float mul = 1.f;
      uint16_t* out;
      if (is_qk) {
        mul = __builtin_amdgcn_rsqf(ss + 1e-6f) * (is_q ? a.scale : 1.f);
        out = is_q ? a.q + ((int64_t)node * a.HK + head) * D : a.k + ((int64_t)node * a.HK + (head - a.HK)) * D;
      } else {
        out = a.v + ((int64_t)node * a.H + (head - 2 * a.HK)) * D;
      }
      u16x8 o;
#pragma unroll
      for (int c = 0; c < CPL; ++c) o[c] = f2bf_bits(y[c] * mul);  // mul == 1 for v heads: y exactly
      if (live) *reinterpret_cast<u16x8*>(out + (cl % D)) = o;
    }
  }
}

// window of node i (request-local indices into [conv state ; request's nodes]), one thread per node
__global__ __launch_bounds__(256) void conv_index_kernel(const int32_t* parents, const int32_t* cu, int R, int N,
                                                         int KC, int32_t* out, int32_t* err) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const int r = cu ? request_of(cu, R, i) : 0;
  const int base = cu ? cu[r] : 0;
  const int nloc = (cu ? cu[r + 1] : N) - base;
  const int li = i - base;
  int32_t* o = out + (int64_t)i * KC;
  o[KC - 1] = KC + li;
  int p = parents[i];
  int last = KC - 1;
  bool bad = false;
  for (int t = KC - 2; t >= 0; --t) {
    if (p >= 0) {
      if (p >= li || p >= nloc) {  // parents must come first
        bad = true;
        p = -1;
        o[t] = last--;
        continue;
      }
      o[t] = KC + p;
      p = parents[base + p];
    } else {
      o[t] = last--;
    }
  }
  if (bad && err) atomicOr(err, MFD_DEVERR_NOT_TOPOLOGICAL);
}

}  // namespace

extern "C" int mfd_conv_index(const int32_t* parents, const int32_t* cu_nodes, int R, int N, int KC,
                              int32_t* conv_index, int32_t* err_flag, void* stream) {
  if (R < 1 || N < 0 || KC < 1 || KC > KC_MAX)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_conv_index: R=%d N=%d KC=%d (1..%d)", R, N, KC, KC_MAX);
  if (N == 0) return MFD_OK;
  if (!parents || !conv_index || (R > 1 && !cu_nodes))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_conv_index: null pointer");
  hipLaunchKernelGGL(conv_index_kernel, dim3((N + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     parents, cu_nodes, R, N, KC, conv_index, err_flag);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

extern "C" int mfd_tree_prep(const uint16_t* x, int64_t x_stride, const uint16_t* conv_state,
                             int64_t conv_state_req_stride, const int32_t* conv_index, const uint16_t* conv_w,
                             const int32_t* cu_nodes, int R, int N, int HK, int H, int D_, int KC, float scale,
                             uint16_t* q_out, uint16_t* k_out, uint16_t* v_out, int32_t* err_flag, void* stream) {
  if (D_ != D) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_tree_prep: head dim %d (only %d)", D_, D);
  if (R < 1 || N < 0 || HK < 1 || H < 1 || KC < 1 || KC > KC_MAX)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_prep: R=%d N=%d HK=%d H=%d KC=%d (1..%d)", R, N, HK, H, KC,
                         KC_MAX);
  const int64_t CD = (int64_t)(2 * HK + H) * D;
  if (x_stride < CD || (x_stride % 8) != 0)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_tree_prep: x row stride %lld (>= %lld, a multiple of 8)",
                         (long long)x_stride, (long long)CD);
  if (N == 0) return MFD_OK;
  if (!x || !conv_state || !conv_index || !conv_w || !q_out || !k_out || !v_out || (R > 1 && !cu_nodes))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_prep: null pointer");
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(conv_state) | reinterpret_cast<uintptr_t>(conv_w) |
        reinterpret_cast<uintptr_t>(q_out) | reinterpret_cast<uintptr_t>(k_out) | reinterpret_cast<uintptr_t>(v_out)) &
       15) != 0 || (conv_state_req_stride % 8) != 0)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_tree_prep: x, conv_state, conv_w and outputs must be 16-byte aligned");
  PrepArgs a{};
  a.x = x; a.x_st = x_stride; a.cs = conv_state; a.cs_rst = conv_state_req_stride; a.cidx = conv_index;
  a.w = conv_w; a.cu = cu_nodes; a.R = R; a.N = N; a.HK = HK; a.H = H; a.scale = scale;
  a.q = q_out; a.k = k_out; a.v = v_out; a.err = err_flag;
  a.hg_blocks = (int)((CD + 4 * 64 * 8 - 1) / (4 * 64 * 8));  // 2048 channels per workgroup
  const int64_t nblocks = (int64_t)((N + NB - 1) / NB) * a.hg_blocks;
  if (nblocks > 0x7FFFFFFF) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_tree_prep: too many nodes x heads");
  const dim3 grid((unsigned)nblocks);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (KC) {
    case 1: hipLaunchKernelGGL(tree_prep_kernel<1>, grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(tree_prep_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 3: hipLaunchKernelGGL(tree_prep_kernel<3>, grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(tree_prep_kernel<4>, grid, dim3(256), 0, st, a); break;
    case 5: hipLaunchKernelGGL(tree_prep_kernel<5>, grid, dim3(256), 0, st, a); break;
    case 6: hipLaunchKernelGGL(tree_prep_kernel<6>, grid, dim3(256), 0, st, a); break;
    case 7: hipLaunchKernelGGL(tree_prep_kernel<7>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(tree_prep_kernel<8>, grid, dim3(256), 0, st, a); break;
  }
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
