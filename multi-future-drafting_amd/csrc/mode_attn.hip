// K-mode drafter attention ("mode attention") for gfx950.
//
// Semantics (inference/hf/mode_attention.py:153-164 reference(); inference/sglang/patches/
// sglang-v0.5.22-mfd.patch:965-988): the K mode blocks of a request sit side by side (K x bs queries,
// mode-major). Query row (head h, query qi) of mode qi / bs attends to every context key of its request
// plus the bs block keys of its own mode (bidirectional inside the block unless causal_in_block);
// query head h reads KV head h / (H / Hkv). Softmax in base 2 with scale * log2(e), fp32 statistics.
//
// Work split: a workgroup takes one (request, KV head, group of 4 units, context split); a unit is 32
// consecutive queries of one query head and runs on one wave. The 4 waves share 64-key K / V tiles staged
// in LDS (double buffered; K as [key][d], V transposed to [d][key] on the way in). Each wave computes
//   S^T = K Q^T   (v_mfma_f32_32x32x16_bf16: A = K rows from LDS, B = Q^T held in registers)
// so a lane owns one query row and the online-softmax rescale is a per-lane scalar, then
//   O^T += V^T P^T (A = V^T rows from LDS, B = P^T straight from the S^T accumulators: the k order of a
//                   16-key chunk is the C-register row order, so no data movement). P is split into bf16
//                   hi + lo (two MFMAs): with near-uniform attention the output is a heavily cancelling
//                   average and a single bf16 rounding of P would cost about 1e-3 of it.
// The request's block keys are processed by the last context split as extra 64-key tiles with the mode
// mask. One split: the normalised output is written as bf16. Several splits: fp32 partials (O / l and
// lse) go to the workspace and a merge kernel combines them (inference/hf/mode_attention.py:91-117).
// Context keys come from a flat layout (slot = position), a per-token slot table (page size 1,
// req_to_token) or a page table (page_size > 1: slot = table[t / P] * P + t % P); context lengths and
// table rows are read on the device, so the launch is graph safe.
#include "mfd_common.h"

namespace {

constexpr int D = 128;
constexpr int TK = 64;        // keys per tile
constexpr int KS_ROW = D + 8; // [key][d] row: 272 B
constexpr int VT_ROW = TK + 4;// [d][key] row: 136 B (b64 reads of 32 consecutive d rows hit distinct banks)
constexpr int NWAVES = 4;
constexpr int NTHREADS = NWAVES * 64;
constexpr int UROWS = 32;     // queries per unit (one wave)

struct alignas(16) AttnSmem {
  uint16_t ks[2][TK][KS_ROW];
  uint16_t vt[2][D][VT_ROW];
};

struct AttnArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kn;
  const uint16_t* vn;
  int64_t kn_st, kn_sh, vn_st, vn_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t kc_ss, kc_sh, vc_ss, vc_sh;
  const int32_t* table;
  int64_t table_stride;
  int page_size;
  const int64_t* req_idx;
  const int64_t* ctx_lens;
  int ctx_const;
  uint16_t* out;
  int64_t o_st, o_sh;
  float* ws_o;    // [S][bs * H * KL][D]
  float* ws_lse;  // [S][bs * H * KL]
  int bs, K, L, H, Hkv, G, S, causal;
  float scale_log2;
  int ngroups;    // unit groups (of NWAVES units) per (request, KV head)
};

__device__ __forceinline__ float wave_xor32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((int)((threadIdx.x & 63) ^ 32) << 2,
                                                              __builtin_bit_cast(int, x)));
}

// Register-staged tile: K chunks for 4 keys (one 16-byte d-chunk each) and V chunks for the same keys.
struct TileRegs {
  u16x8 k[4];
  u16x8 v[4];
};

__global__ __launch_bounds__(NTHREADS) void mode_attn_kernel(AttnArgs a) {
  __shared__ AttnSmem sm;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int KL = a.K * a.L;

  // ---- workgroup -> (request b, KV head, unit group, split); the unit groups of one (b, KV head, split)
  //      read the same K / V chunk and share an XCD (workgroup id modulo 8)
  const int P = a.bs * a.Hkv * a.S;
  const int P8 = (P + 7) >> 3;
  const int id = blockIdx.x;
  const int rest = id >> 3;
  const int pidx = (rest % P8) * 8 + (id & 7);
  if (pidx >= P) return;
  const int ug = rest / P8;
  const int s = pidx % a.S;
  const int bk = pidx / a.S;
  const int kvh = bk % a.Hkv;
  const int b = bk / a.Hkv;

  const int upr = KL / UROWS;              // units per query head
  const int U = a.G * upr;
  const int u = ug * NWAVES + w;
  const bool active = u < U;
  const int g = active ? u / upr : 0;
  const int head = kvh * a.G + g;
  const int qi = (active ? (u % upr) * UROWS : 0) + l32;  // this lane's query row
  const int token = b * KL + qi;
  const int mode = qi / a.L;
  const int tpos = qi % a.L;

  // Q^T fragments: B operand, k = d = 16c + 8 half + e
  bf16x8 qf[D / 16];
  {
    const uint16_t* qp = a.q + (int64_t)token * a.q_st + (int64_t)head * a.q_sh + half * 8;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qf[c] = as_bf16x8(*reinterpret_cast<const u16x8*>(qp + c * 16));
  }

  const int ctx = a.ctx_lens ? (int)a.ctx_lens[b] : a.ctx_const;
  const int64_t trow = a.req_idx ? a.req_idx[b] : b;
  int lo = 0, hi = ctx;
  if (a.S > 1) {
    const int per = (ctx + a.S - 1) / a.S;
    const int chunk = max(TK, (per + TK - 1) / TK * TK);
    lo = s * chunk;
    hi = min(lo + chunk, ctx);
    if (lo > hi) lo = hi;
  }
  const int n_ctx_tiles = (hi - lo + TK - 1) / TK;
  const int n_blk_tiles = (s == a.S - 1) ? (KL + TK - 1) / TK : 0;
  const int ntiles = n_ctx_tiles + n_blk_tiles;

  // tile loader: thread -> keys 4 kg .. 4 kg + 3 (kg = tid / 16), d chunk dc = tid % 16
  const int kg = tid >> 4;
  const int dc = tid & 15;
  auto load_tile = [&](int t, TileRegs& tr) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int j = kg * 4 + x;
      const uint16_t* kp;
      const uint16_t* vp;
      bool ok;
      if (t < n_ctx_tiles) {
        const int key = lo + t * TK + j;
        ok = key < hi;
        const int kk = ok ? key : lo;
        int64_t slot = kk;
        if (a.table) {
          if (a.page_size == 1) {
            slot = a.table[trow * a.table_stride + kk];
          } else {
            slot = (int64_t)a.table[trow * a.table_stride + kk / a.page_size] * a.page_size + kk % a.page_size;
          }
        }
        kp = a.kc + slot * a.kc_ss + (int64_t)kvh * a.kc_sh;
        vp = a.vc + slot * a.vc_ss + (int64_t)kvh * a.vc_sh;
      } else {
        const int key = (t - n_ctx_tiles) * TK + j;
        ok = key < KL;
        const int64_t tk = (int64_t)b * KL + (ok ? key : 0);
        kp = a.kn + tk * a.kn_st + (int64_t)kvh * a.kn_sh;
        vp = a.vn + tk * a.vn_st + (int64_t)kvh * a.vn_sh;
      }
      if (ctx == 0 && t < n_ctx_tiles) ok = false;
      tr.k[x] = *reinterpret_cast<const u16x8*>(kp + dc * 8);
      tr.v[x] = *reinterpret_cast<const u16x8*>(vp + dc * 8);
      if (!ok) {
        tr.k[x] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
        tr.v[x] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int buf, const TileRegs& tr) {
#pragma unroll
    for (int x = 0; x < 4; ++x) *reinterpret_cast<u16x8*>(&sm.ks[buf][kg * 4 + x][dc * 8]) = tr.k[x];
    // V^T: for each of the 8 d of the chunk, the 4 keys are contiguous
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const u16x4 col = {tr.v[0][e], tr.v[1][e], tr.v[2][e], tr.v[3][e]};
      *reinterpret_cast<u16x4*>(&sm.vt[buf][dc * 8 + e][kg * 4]) = col;
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 oacc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) oacc[db] = (f32x16){};

  TileRegs tr;
  if (ntiles > 0) {
    load_tile(0, tr);
    store_tile(0, tr);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1, tr);
    if (active) {
      // S^T subtiles: keys 32 ks + 8 (r / 4) + 4 half + r % 4 of the tile, column = this lane's query
      f32x16 sv[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        f32x16 acc = {};
#pragma unroll
        for (int c = 0; c < D / 16; ++c)
          acc = mfma32(as_bf16x8(*reinterpret_cast<const u16x8*>(&sm.ks[buf][ks * 32 + l32][c * 16 + half * 8])), qf[c],
                       acc);
        sv[ks] = acc;
      }
      const bool is_ctx = t < n_ctx_tiles;
      const int base = is_ctx ? lo + t * TK : (t - n_ctx_tiles) * TK;
      const int lim = is_ctx ? hi : KL;
      float tmax = -INFINITY;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = base + ks * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          bool ok = key < lim;
          if (!is_ctx) {
            ok = ok && (key / a.L == mode);
            if (a.causal) ok = ok && (key % a.L <= tpos);
          }
          const float x = ok ? sv[ks][r] * a.scale_log2 : -INFINITY;
          sv[ks][r] = x;
          tmax = fmaxf(tmax, x);
        }
      tmax = fmaxf(tmax, wave_xor32(tmax));
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
      const float msub = (m_new == -INFINITY) ? 0.f : m_new;
      // P^T as B fragments, split into bf16 hi + lo so that the PV product keeps fp32-level weights
      float psum = 0.f;
      bf16x8 pf[4], pl[4];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = exp2f(sv[ks][r] - msub);
          psum += p;
          __bf16 hi, lo;
          split_bf16(p, hi, lo);
          pf[ks * 2 + (r >> 3)][r & 7] = hi;
          pl[ks * 2 + (r >> 3)][r & 7] = lo;
        }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        f32x16 o = oacc[db] * alpha;
#pragma unroll
        for (int c = 0; c < TK / 16; ++c) {
          const u16x4 x0 = *reinterpret_cast<const u16x4*>(&sm.vt[buf][db * 32 + l32][c * 16 + half * 4]);
          const u16x4 x1 = *reinterpret_cast<const u16x4*>(&sm.vt[buf][db * 32 + l32][c * 16 + 8 + half * 4]);
          const u16x8 va = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          o = mfma32(as_bf16x8(va), pf[c], o);
          o = mfma32(as_bf16x8(va), pl[c], o);
        }
        oacc[db] = o;
      }
    }
    if (t + 1 < ntiles) store_tile(buf ^ 1, tr);
    __syncthreads();
  }
  if (!active) return;

  const float l_tot = l_run + wave_xor32(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (a.S == 1) {
    uint16_t* op = a.out + (int64_t)token * a.o_st + (int64_t)head * a.o_sh;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = db * 32 + gq * 8 + half * 4;
        const u16x4 vals = {f2bf_bits(oacc[db][gq * 4 + 0] * inv), f2bf_bits(oacc[db][gq * 4 + 1] * inv),
                            f2bf_bits(oacc[db][gq * 4 + 2] * inv), f2bf_bits(oacc[db][gq * 4 + 3] * inv)};
        *reinterpret_cast<u16x4*>(op + d0) = vals;
      }
  } else {
    const int64_t prow = ((int64_t)b * a.H + head) * KL + qi;
    const int64_t nrows = (int64_t)a.bs * a.H * KL;
    float* op = a.ws_o + ((int64_t)s * nrows + prow) * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = db * 32 + gq * 8 + half * 4;
        const f32x4 vals = {oacc[db][gq * 4 + 0] * inv, oacc[db][gq * 4 + 1] * inv, oacc[db][gq * 4 + 2] * inv,
                            oacc[db][gq * 4 + 3] * inv};
        *reinterpret_cast<f32x4*>(op + d0) = vals;
      }
    if (half == 0) a.ws_lse[(int64_t)s * nrows + prow] = l_tot > 0.f ? m_run + __log2f(l_tot) : -INFINITY;
  }
}

// one thread per 4 d of one row; 32 threads per row
__global__ __launch_bounds__(256) void mode_attn_merge_kernel(AttnArgs a) {
  const int KL = a.K * a.L;
  const int64_t nrows = (int64_t)a.bs * a.H * KL;
  const int64_t prow = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (prow >= nrows) return;
  const int d0 = (threadIdx.x & 31) * 4;
  float m = -INFINITY;
  for (int s = 0; s < a.S; ++s) m = fmaxf(m, a.ws_lse[s * nrows + prow]);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float tot = 0.f;
  if (m != -INFINITY) {
    for (int s = 0; s < a.S; ++s) {
      const float lse = a.ws_lse[s * nrows + prow];
      if (lse == -INFINITY) continue;
      const float wgt = exp2f(lse - m);
      const f32x4 o = *reinterpret_cast<const f32x4*>(a.ws_o + (s * nrows + prow) * D + d0);
      acc += o * wgt;
      tot += wgt;
    }
  }
  const float inv = tot > 0.f ? 1.f / tot : 0.f;
  const int qi = (int)(prow % KL);
  const int64_t bh = prow / KL;
  const int head = (int)(bh % a.H);
  const int b = (int)(bh / a.H);
  uint16_t* op = a.out + ((int64_t)b * KL + qi) * a.o_st + (int64_t)head * a.o_sh + d0;
  const u16x4 vals = {f2bf_bits(acc[0] * inv), f2bf_bits(acc[1] * inv), f2bf_bits(acc[2] * inv), f2bf_bits(acc[3] * inv)};
  *reinterpret_cast<u16x4*>(op) = vals;
}

}  // namespace

extern "C" int64_t mfd_mode_attn_workspace_bytes(int bs, int num_modes, int block_size, int H, int num_ctx_splits) {
  if (num_ctx_splits <= 1) return 0;
  const int64_t rows = (int64_t)bs * H * num_modes * block_size;
  return (int64_t)num_ctx_splits * rows * (D + 1) * (int64_t)sizeof(float);
}

extern "C" int mfd_mode_attn(const uint16_t* q, int64_t q_st, int64_t q_sh, const uint16_t* k_new,
                             const uint16_t* v_new, int64_t kn_st, int64_t kn_sh, int64_t vn_st, int64_t vn_sh,
                             const uint16_t* k_cache, const uint16_t* v_cache, int64_t kc_ss, int64_t kc_sh,
                             int64_t vc_ss, int64_t vc_sh, const int32_t* slot_table, int64_t table_stride,
                             int page_size, const int64_t* req_idx, const int64_t* ctx_lens, int ctx_len_const, int bs,
                             int num_modes, int block_size, int H, int Hkv, int D_, float scale, int causal_in_block,
                             int num_ctx_splits, uint16_t* out, int64_t o_st, int64_t o_sh, float* workspace,
                             int64_t workspace_bytes, void* stream) {
  if (D_ != D) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_mode_attn: head dim %d (only %d)", D_, D);
  if (bs < 0 || num_modes < 1 || block_size < 1 || H < 1 || Hkv < 1 || H % Hkv != 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: bad sizes bs=%d K=%d L=%d H=%d Hkv=%d", bs, num_modes,
                         block_size, H, Hkv);
  const int KL = num_modes * block_size;
  if (KL % UROWS != 0)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_mode_attn: num_modes * block_size = %d must be a multiple of %d", KL,
                         UROWS);
  if (num_ctx_splits < 1 || num_ctx_splits > 1024)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: num_ctx_splits %d (1..1024)", num_ctx_splits);
  if (page_size < 1) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: page_size %d", page_size);
  if (!ctx_lens && ctx_len_const < 0) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: negative context length");
  if (bs == 0) return MFD_OK;
  if (!q || !k_new || !v_new || !out || ((!k_cache || !v_cache) && (ctx_lens || ctx_len_const > 0)))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: null tensor pointer");
  const int64_t need = mfd_mode_attn_workspace_bytes(bs, num_modes, block_size, H, num_ctx_splits);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: workspace of %lld bytes needed", (long long)need);
  AttnArgs a{};
  a.q = q; a.q_st = q_st; a.q_sh = q_sh;
  a.kn = k_new; a.vn = v_new; a.kn_st = kn_st; a.kn_sh = kn_sh; a.vn_st = vn_st; a.vn_sh = vn_sh;
  a.kc = k_cache; a.vc = v_cache; a.kc_ss = kc_ss; a.kc_sh = kc_sh; a.vc_ss = vc_ss; a.vc_sh = vc_sh;
  a.table = slot_table; a.table_stride = table_stride; a.page_size = page_size;
  a.req_idx = req_idx; a.ctx_lens = ctx_lens; a.ctx_const = ctx_len_const;
  a.out = out; a.o_st = o_st; a.o_sh = o_sh;
  const int64_t rows = (int64_t)bs * H * KL;
  a.ws_o = workspace;
  a.ws_lse = workspace ? workspace + (int64_t)num_ctx_splits * rows * D : nullptr;
  a.bs = bs; a.K = num_modes; a.L = block_size; a.H = H; a.Hkv = Hkv; a.G = H / Hkv; a.S = num_ctx_splits;
  a.causal = causal_in_block ? 1 : 0;
  a.scale_log2 = scale * 1.4426950408889634f;
  const int units = a.G * (KL / UROWS);
  a.ngroups = (units + NWAVES - 1) / NWAVES;
  const int P = bs * Hkv * num_ctx_splits;
  const int P8 = (P + 7) / 8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(mode_attn_kernel, dim3(8 * P8 * a.ngroups), dim3(NTHREADS), 0, st, a);
  MFD_CHECK_LAUNCH();
  if (num_ctx_splits > 1) {
    hipLaunchKernelGGL(mode_attn_merge_kernel, dim3((unsigned)((rows + 7) / 8)), dim3(256), 0, st, a);
    MFD_CHECK_LAUNCH();
  }
  return MFD_OK;
}
