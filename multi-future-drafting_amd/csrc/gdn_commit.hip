// Commit of a verified tree for gfx950: every GDN layer's recurrent state and conv state advance to the
// deepest accepted node a (inference/hf/qwen35_tree.py:122-148 commit), all layers in one launch:
//
//   S_l,h <- exp(G_l[a,h]) S_l,h + sum_{j on the accepted path} exp(G_l[a,h] - G_l[j,h]) k_l[j, h / (H / HK)] u_l[j,h]^T
//   conv_l[c][t] <- window_t(c) of node a: conv_l[c][idx] (old state) if idx < KC, else x_l[idx - KC][c]
//
// (S in the [d_k, d_v] layout, fp32, updated in place; u, k, G, x are the verify pass's per-layer values.)
// One workgroup per (layer, value head) for the state: it streams its 64 KB slice once (read, update,
// write; HBM-bound), with the accepted nodes' scaled keys e^{G_a - G_j} k_j and u_j staged in LDS 32 at a
// time (for paths of at most 32 nodes, before the state is requested, and the state then updated and stored
// in two halves); thread t owns four value columns of 16 key rows. Further workgroups rewrite the conv states, one
// thread per channel of a layer (the KC old columns are read before any is written, so in place is safe).
#include "mfd_common.h"

namespace {

constexpr int D = 128;
constexpr int PCH = 32;    // accepted nodes staged per pass
constexpr int KC_MAX = 8;

struct CommitArgs {
  float* S;            // [L][H][D][D]
  int64_t s_lst;
  const float* u;      // [L][n][H][D]
  int64_t u_lst;
  const uint16_t* k;   // [L][n][HK][D]
  int64_t k_lst;
  const float* G;      // [L][n][H]
  int64_t g_lst;
  const int32_t* path; // [p] node ids, root first
  int p, L, n, HK, H;
  uint16_t* conv;      // [L][CD][KC] or null
  int64_t c_lst;
  const uint16_t* x;   // [L][n][CD], row stride x_rst
  int64_t x_lst, x_rst;
  const int32_t* cidx; // [n][KC]
  int CD, KC, conv_blocks;
  int32_t* err;
};

__device__ __forceinline__ bool valid_node(int j, int n) { return j >= 0 && j < n; }

__global__ __launch_bounds__(256) void gdn_commit_kernel(CommitArgs a) {
  __shared__ float wk[PCH][D];  // e^{G_a - G_j} k_j
  __shared__ float us[PCH][D];  // u_j
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int last = a.path[a.p - 1];
  if (!valid_node(last, a.n)) {  // nothing is written for an invalid path end
    if (tid == 0 && a.err) atomicOr(a.err, MFD_DEVERR_BAD_WINDOW);
    return;
  }
  if (b < a.L * a.H) {
    const int l = b / a.H, h = b % a.H;
    const int hk = h / (a.H / a.HK);
    const float* Gl = a.G + (int64_t)l * a.g_lst;
    const float Ga = Gl[(int64_t)last * a.H + h];
    const float ea = __expf(Ga);
    float* S = a.S + (int64_t)l * a.s_lst + (int64_t)h * D * D;
    const int col = (tid & 31) * 4;
    const int r0 = tid >> 5;
    const float* ul = a.u + (int64_t)l * a.u_lst;
    const uint16_t* kl = a.k + (int64_t)l * a.k_lst;
    // stage the scaled keys and u rows of path nodes j0 .. j0 + np - 1
    auto stage = [&](int j0, int np) {
      for (int e = tid; e < np * D; e += 256) {
        const int j = e / D, d = e % D;
        const int node = a.path[j0 + j];
        float w = 0.f, uu = 0.f;
        if (valid_node(node, a.n)) {
          w = __expf(Ga - Gl[(int64_t)node * a.H + h]) * bf2f(kl[((int64_t)node * a.HK + hk) * D + d]);
          uu = ul[((int64_t)node * a.H + h) * D + d];
        } else if (a.err) {
          atomicOr(a.err, MFD_DEVERR_BAD_WINDOW);
        }
        wk[j][d] = w;
        us[j][d] = uu;
      }
    };
    f32x4 acc[D / 8];
    if (a.p <= PCH) {
      // the path's rows are staged before the state is requested (their dependent loads would otherwise queue
      // behind the 64 KB of state), and the state is updated and stored in two halves of 64 key rows, the
      // first half's stores draining while the second half is computed
      stage(0, a.p);
      __syncthreads();
#pragma unroll
      for (int m = 0; m < D / 8; ++m) acc[m] = *reinterpret_cast<const f32x4*>(S + (r0 + 8 * m) * D + col);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
        for (int m = 8 * hf; m < 8 * hf + 8; ++m) acc[m] *= ea;
        for (int j = 0; j < a.p; ++j) {
          const f32x4 uu = *reinterpret_cast<const f32x4*>(&us[j][col]);
#pragma unroll
          for (int m = 8 * hf; m < 8 * hf + 8; ++m) acc[m] += wk[j][r0 + 8 * m] * uu;
        }
#pragma unroll
        for (int m = 8 * hf; m < 8 * hf + 8; ++m) *reinterpret_cast<f32x4*>(S + (r0 + 8 * m) * D + col) = acc[m];
      }
      return;
    }
#pragma unroll
    for (int m = 0; m < D / 8; ++m) acc[m] = ea * *reinterpret_cast<const f32x4*>(S + (r0 + 8 * m) * D + col);
    for (int j0 = 0; j0 < a.p; j0 += PCH) {
      const int np = min(PCH, a.p - j0);
      __syncthreads();
      stage(j0, np);
      __syncthreads();
      for (int j = 0; j < np; ++j) {
        const f32x4 uu = *reinterpret_cast<const f32x4*>(&us[j][col]);
#pragma unroll
        for (int m = 0; m < D / 8; ++m) acc[m] += wk[j][r0 + 8 * m] * uu;
      }
    }
#pragma unroll
    for (int m = 0; m < D / 8; ++m) *reinterpret_cast<f32x4*>(S + (r0 + 8 * m) * D + col) = acc[m];
    return;
  }
  // conv state of layer l, channel c
  const int cb = b - a.L * a.H;
  const int l = cb / a.conv_blocks;
  const int c = (cb % a.conv_blocks) * 256 + tid;
  if (l >= a.L || c >= a.CD) return;
  const int KC = a.KC;
  uint16_t* cv = a.conv + (int64_t)l * a.c_lst + (int64_t)c * KC;
  const uint16_t* xl = a.x + (int64_t)l * a.x_lst;
  uint16_t val[KC_MAX];
#pragma unroll
  for (int t = 0; t < KC_MAX; ++t) {
    if (t < KC) {
      const int idx = a.cidx[(int64_t)last * KC + t];
      uint16_t v = 0;
      if (idx >= 0 && idx < KC) {
        v = cv[idx];
      } else if (idx >= KC && idx - KC < a.n) {
        v = xl[(int64_t)(idx - KC) * a.x_rst + c];
      } else if (a.err) {
        atomicOr(a.err, MFD_DEVERR_BAD_WINDOW);
      }
      val[t] = v;
    }
  }
#pragma unroll
  for (int t = 0; t < KC_MAX; ++t)
    if (t < KC) cv[t] = val[t];
}

}  // namespace

extern "C" int mfd_gdn_commit(float* state, int64_t state_layer_stride, const float* u, int64_t u_layer_stride,
                              const uint16_t* k, int64_t k_layer_stride, const float* g_cum, int64_t g_layer_stride,
                              const int32_t* path, int p, int L, int n, int HK, int H, int D_, uint16_t* conv,
                              int64_t conv_layer_stride, const uint16_t* x, int64_t x_layer_stride,
                              int64_t x_row_stride, const int32_t* conv_index, int CD, int KC, int32_t* err_flag,
                              void* stream) {
  if (D_ != D) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_gdn_commit: head dim %d (only %d)", D_, D);
  if (L < 0 || n < 1 || p < 1 || p > n || HK < 1 || H < 1 || H % HK != 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_gdn_commit: L=%d n=%d p=%d HK=%d H=%d", L, n, p, HK, H);
  if (conv && (KC < 1 || KC > KC_MAX || CD < 1))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_gdn_commit: conv state with KC=%d (1..%d) CD=%d", KC, KC_MAX, CD);
  if (L == 0) return MFD_OK;
  if (!state || !u || !k || !g_cum || !path || (conv && (!x || !conv_index)))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_gdn_commit: null pointer");
  if ((reinterpret_cast<uintptr_t>(state) & 15) != 0 || (state_layer_stride % 4) != 0 ||
      (reinterpret_cast<uintptr_t>(u) & 15) != 0 || (u_layer_stride % 4) != 0)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_gdn_commit: state and u must be 16-byte aligned per layer");
  CommitArgs a{};
  a.S = state; a.s_lst = state_layer_stride; a.u = u; a.u_lst = u_layer_stride; a.k = k; a.k_lst = k_layer_stride;
  a.G = g_cum; a.g_lst = g_layer_stride; a.path = path; a.p = p; a.L = L; a.n = n; a.HK = HK; a.H = H;
  a.conv = conv; a.c_lst = conv_layer_stride; a.x = x; a.x_lst = x_layer_stride; a.x_rst = x_row_stride;
  a.cidx = conv_index; a.CD = CD; a.KC = KC; a.err = err_flag;
  a.conv_blocks = conv ? (CD + 255) / 256 : 0;
  const int64_t nblocks = (int64_t)L * H + (int64_t)L * a.conv_blocks;
  hipLaunchKernelGGL(gdn_commit_kernel, dim3((unsigned)nblocks), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
