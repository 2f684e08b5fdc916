// Tree gated-delta-rule verification for gfx950 — one workgroup per (request, value head).
//
// Math (inference/hf/tree_gdn_kernel.py:3-6, inference/hf/qwen35_tree.py:9-20). For the nodes of one tree
// in topological order, with A_ij = beta_i e^{G_i-G_j} k_i.k_j on strict ancestors and
// P_ij = e^{G_i-G_j} q_i.k_j on ancestors-or-self:
//   u = (I + A)^{-1} R,  R_i = beta_i (v_i - e^{G_i} S0^T k_i)
//   o = E + P u,         E_i = e^{G_i} S0^T q_i
// Instead of block inverses over dense n x n blocks, the kernel uses the tree structure: the
// non-zeros of row i of T = (I + A)^{-1} sit on i's root path (at most MAXD entries), and each
// row is obtained by a path-local back substitution T_i[s] = -sum_{m>s} T_i[m] A_{path(i,m), path(i,s)}.
// With W = P T (also path-supported), u = T R and o = E + W R. All dense products run on MFMA
// (v_mfma_f32_32x32x16_bf16) with fp32 operands split into bf16 hi + lo pairs:
//   phase 1  Gram entries k_i.k_j, q_i.k_j of the lower tiles, kept only for ancestor pairs
//   phase 2  path coefficients a, p; phase 3 rows of T; phase 4 rows of W (VALU, per node)
//   phase 5  K S0 and Q S0 (S0 split hi/lo) -> R (split hi/lo, kept in registers) and E
//   phase 6  per 32-row block: dense T / W rows staged in LDS, u = T R, o = E + W R, stores.
// The R accumulators of phase 5 are fed straight back as the B operand of phase 6: the k order of
// a 16-node chunk is chosen to be the C-register row order (rows 16c + 4h + e and 16c + 8 + 4h + e
// for lane half h), so no cross-lane movement is needed.
#include "mfd_common.h"

namespace {

constexpr int D = MFD_GDN_HEAD_DIM;   // 128
constexpr int MAXD = MFD_GDN_MAX_DEPTH;
constexpr int KROW = D + 8;           // padded LDS row of K / Q (272 B: rows shift by 4 banks)
constexpr int NTHREADS = 256;         // 4 waves; wave w owns value columns [32w, 32w + 32)

template <int NT>
struct GdnSmem {
  static constexpr int NMAX = 32 * NT;
  static constexpr int SROW = NMAX + 8;   // padded staged row (bf16 elements)
  uint16_t kq[2][NMAX][KROW];             // K rows, Q rows of this request / key head
  uint16_t stage[2][2][32][SROW];         // [T or W][hi or lo][row in block][node]
  float coefA[NMAX][MAXD];                // k_i.k_j -> a_ij -> W_ij
  float coefP[NMAX][MAXD];                // q_i.k_j -> p_ij
  float coefT[NMAX][MAXD];                // T_ij
  int16_t path[NMAX][MAXD];               // path[i][s] = ancestor of i at depth s + 1 (path[i][depth-1] = i)
  int par[NMAX];
  int depth[NMAX];
  float G[NMAX], beta[NMAX], eG[NMAX];
  int bad;
};

struct GdnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* g_cum;
  const float* beta;
  const float* s0;
  const int32_t* parents;
  const int8_t* anc8;
  const int32_t* cu_nodes;
  float* u;
  float* o;
  int32_t* err;
  int R, N, HK, H;
};

template <int NT>
__global__ __launch_bounds__(NTHREADS) void tree_gdn_kernel(GdnArgs a) {
  using S = GdnSmem<NT>;
  constexpr int NMAX = S::NMAX;
  __shared__ S sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;

  // ---- XCD-aware mapping: the G value heads of one (request, key head) share q/k, keep them on one XCD.
  const int G = a.H / a.HK;
  const int P = a.R * a.HK;
  const int P8 = (P + 7) >> 3;
  const int id = blockIdx.x;
  const int xcd = id & 7;
  const int rest = id >> 3;
  const int slot = rest % P8;
  const int gq = rest / P8;
  const int pidx = slot * 8 + xcd;
  if (pidx >= P) return;
  const int r = pidx / a.HK;
  const int hk = pidx % a.HK;
  const int h = hk * G + gq;

  const int ns = a.cu_nodes ? a.cu_nodes[r] : 0;
  const int n = a.cu_nodes ? a.cu_nodes[r + 1] - ns : a.N;
  if (n <= 0) return;
  if (n > NMAX) {
    if (tid == 0 && a.err) atomicOr(a.err, MFD_DEVERR_TOO_MANY_NODES);
    return;
  }
  const int nt = (n + 31) >> 5;

  // ---- phase 0: tree metadata, gates, K/Q rows into LDS
  if (tid == 0) sm.bad = 0;
  for (int i = tid; i < NMAX; i += NTHREADS) {
    int p = -1;
    if (i < n) {
      if (a.parents) {
        p = a.parents[ns + i];
      } else {
        const int8_t* row = a.anc8 + (size_t)i * n;
        for (int j = i - 1; j >= 0; --j)
          if (row[j] != 0) { p = j; break; }
      }
      const float gg = a.g_cum[(size_t)(ns + i) * a.H + h];
      sm.G[i] = gg;
      sm.eG[i] = __expf(gg);
      sm.beta[i] = a.beta[(size_t)(ns + i) * a.H + h];
    } else {
      sm.G[i] = 0.f;
      sm.eG[i] = 0.f;
      sm.beta[i] = 0.f;
    }
    sm.par[i] = p;
  }
  {
    // 16-byte chunks: NMAX rows x 16 chunks, for K then Q
    const uint16_t* srcs[2] = {a.k, a.q};
    for (int t = tid; t < 2 * NMAX * (D / 8); t += NTHREADS) {
      const int which = t / (NMAX * (D / 8));
      const int rem = t % (NMAX * (D / 8));
      const int i = rem / (D / 8);
      const int c8 = rem % (D / 8);
      u16x8 val = {0, 0, 0, 0, 0, 0, 0, 0};
      if (i < n) val = *reinterpret_cast<const u16x8*>(srcs[which] + ((size_t)(ns + i) * a.HK + hk) * D + c8 * 8);
      *reinterpret_cast<u16x8*>(&sm.kq[which][i][c8 * 8]) = val;
    }
  }
  __syncthreads();
  for (int i = tid; i < NMAX; i += NTHREADS) {
    int d = 0;
    if (i < n) {
      int cur = i;
      while (cur >= 0 && d <= MAXD) {
        const int p = sm.par[cur];
        if (p >= cur) { atomicOr(&sm.bad, MFD_DEVERR_NOT_TOPOLOGICAL); break; }
        ++d;
        cur = p;
      }
      if (d > MAXD) atomicOr(&sm.bad, MFD_DEVERR_TOO_DEEP);
      if (d <= MAXD) {
        cur = i;
        for (int s = d - 1; s >= 0 && cur >= 0; --s) {
          sm.path[i][s] = (int16_t)cur;
          cur = sm.par[cur];
        }
      }
    }
    sm.depth[i] = d;
    for (int s = 0; s < MAXD; ++s) {
      sm.coefA[i][s] = 0.f;
      sm.coefP[i][s] = 0.f;
      sm.coefT[i][s] = 0.f;
    }
  }
  __syncthreads();
  if (sm.bad) {
    if (tid == 0 && a.err) atomicOr(a.err, sm.bad);
    return;
  }

  // ---- phase 1: Gram entries on ancestor pairs (lower 32x32 tiles, distributed over the 4 waves)
  {
    const int ntiles = nt * (nt + 1) / 2;
    for (int t = w; t < ntiles; t += 4) {
      int ib = 0;
      while ((ib + 1) * (ib + 2) / 2 <= t) ++ib;
      const int jb = t - ib * (ib + 1) / 2;
      f32x16 akk = {}, aqk = {};
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        const int kof = c * 16 + half * 8;
        const bf16x8 ak = as_bf16x8(*reinterpret_cast<const u16x8*>(&sm.kq[0][ib * 32 + l32][kof]));
        const bf16x8 aq = as_bf16x8(*reinterpret_cast<const u16x8*>(&sm.kq[1][ib * 32 + l32][kof]));
        const bf16x8 bk = as_bf16x8(*reinterpret_cast<const u16x8*>(&sm.kq[0][jb * 32 + l32][kof]));
        akk = mfma32(ak, bk, akk);
        aqk = mfma32(aq, bk, aqk);
      }
      const int j = jb * 32 + l32;
      const int dj = sm.depth[j];
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int i = ib * 32 + 8 * (rr >> 2) + 4 * half + (rr & 3);
        if (i < n && j <= i && dj > 0 && dj <= sm.depth[i] && sm.path[i][dj - 1] == j) {
          sm.coefP[i][dj - 1] = aqk[rr];
          if (j < i) sm.coefA[i][dj - 1] = akk[rr];
        }
      }
    }
  }
  __syncthreads();

  // ---- phase 2: a_ij = beta_i e^{G_i-G_j} k_i.k_j (strict), p_ij = e^{G_i-G_j} q_i.k_j
  if (tid < n) {
    const int i = tid;
    const int d = sm.depth[i];
    const float gi = sm.G[i];
    const float bi = sm.beta[i];
    for (int s = 0; s < d; ++s) {
      const int j = sm.path[i][s];
      const float e = __expf(gi - sm.G[j]);
      sm.coefP[i][s] *= e;
      if (s < d - 1) sm.coefA[i][s] *= bi * e;
    }
  }
  __syncthreads();
  // ---- phase 3: rows of T = (I + A)^{-1} by path-local back substitution
  if (tid < n) {
    const int i = tid;
    const int d = sm.depth[i];
    sm.coefT[i][d - 1] = 1.f;
    for (int s = d - 2; s >= 0; --s) {
      float acc = 0.f;
      for (int m = s + 1; m < d; ++m) acc += sm.coefT[i][m] * sm.coefA[sm.path[i][m]][s];
      sm.coefT[i][s] = -acc;
    }
  }
  __syncthreads();
  // ---- phase 4: rows of W = P T (stored over coefA, whose values T no longer needs)
  float wrow[MAXD];
  if (tid < n) {
    const int i = tid;
    const int d = sm.depth[i];
#pragma unroll
    for (int s = 0; s < MAXD; ++s) {
      float acc = 0.f;
      if (s < d)
        for (int m = s; m < d; ++m) acc += sm.coefP[i][m] * sm.coefT[sm.path[i][m]][s];
      wrow[s] = acc;
    }
  }
  __syncthreads();
  if (tid < n) {
#pragma unroll
    for (int s = 0; s < MAXD; ++s) sm.coefA[tid][s] = wrow[s];
  }
  // (the barrier of phase 6's first staging round orders these writes before their reads)

  // ---- phase 5: K S0, Q S0 with S0 split hi/lo -> R (hi/lo, registers) and E (o accumulators)
  const int vcol = w * 32 + l32;
  const size_t rh = (size_t)r * a.H + h;
  bf16x8 Rb[NT][2][2];      // [row tile][16-node chunk][hi, lo]
  f32x16 oacc[NT];
  {
    bf16x8 sh[D / 16], sl[D / 16];
    const float* s0p = a.s0 + rh * D * D + vcol;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = s0p[(size_t)(c * 16 + half * 8 + e) * D];
        __bf16 hi, lo;
        split_bf16(x, hi, lo);
        sh[c][e] = hi;
        sl[c][e] = lo;
      }
    }
#pragma unroll
    for (int ib = 0; ib < NT; ++ib) {
      f32x16 ak = {}, aq = {};
      if (ib < nt) {
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          const int kof = c * 16 + half * 8;
          const bf16x8 fk = as_bf16x8(*reinterpret_cast<const u16x8*>(&sm.kq[0][ib * 32 + l32][kof]));
          const bf16x8 fq = as_bf16x8(*reinterpret_cast<const u16x8*>(&sm.kq[1][ib * 32 + l32][kof]));
          ak = mfma32(fk, sh[c], ak);
          ak = mfma32(fk, sl[c], ak);
          aq = mfma32(fq, sh[c], aq);
          aq = mfma32(fq, sl[c], aq);
        }
      }
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int i = ib * 32 + 8 * (rr >> 2) + 4 * half + (rr & 3);
        float rv = 0.f, ev = 0.f;
        if (i < n) {
          const float vv = bf2f(a.v[((size_t)(ns + i) * a.H + h) * D + vcol]);
          rv = sm.beta[i] * (vv - sm.eG[i] * ak[rr]);
          ev = sm.eG[i] * aq[rr];
        }
        __bf16 hi, lo;
        split_bf16(rv, hi, lo);
        Rb[ib][rr >> 3][0][rr & 7] = hi;
        Rb[ib][rr >> 3][1][rr & 7] = lo;
        oacc[ib][rr] = ev;
      }
    }
  }

  // ---- phase 6: per 32-row block, dense T / W rows in LDS, u = T R, o = E + W R
#pragma unroll
  for (int ib = 0; ib < NT; ++ib) {
    if (ib >= nt) break;
    const int ncols = 32 * (ib + 1);
    __syncthreads();  // previous block's staged rows are consumed (and phase 4's writes are visible)
    // gather: item = (row in block, 8-column chunk)
    for (int t = tid; t < 32 * (ncols / 8); t += NTHREADS) {
      const int rl = t / (ncols / 8);
      const int c8 = t % (ncols / 8);
      const int i = ib * 32 + rl;
      u16x8 th = {}, tl = {}, wh = {}, wl = {};
      if (i < n) {
        const int di = sm.depth[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = c8 * 8 + e;
          if (j <= i) {
            const int dj = sm.depth[j];
            if (dj > 0 && dj <= di && sm.path[i][dj - 1] == j) {
              __bf16 hi, lo;
              split_bf16(sm.coefT[i][dj - 1], hi, lo);
              th[e] = __builtin_bit_cast(uint16_t, hi);
              tl[e] = __builtin_bit_cast(uint16_t, lo);
              split_bf16(sm.coefA[i][dj - 1], hi, lo);
              wh[e] = __builtin_bit_cast(uint16_t, hi);
              wl[e] = __builtin_bit_cast(uint16_t, lo);
            }
          }
        }
      }
      *reinterpret_cast<u16x8*>(&sm.stage[0][0][rl][c8 * 8]) = th;
      *reinterpret_cast<u16x8*>(&sm.stage[0][1][rl][c8 * 8]) = tl;
      *reinterpret_cast<u16x8*>(&sm.stage[1][0][rl][c8 * 8]) = wh;
      *reinterpret_cast<u16x8*>(&sm.stage[1][1][rl][c8 * 8]) = wl;
    }
    __syncthreads();
    f32x16 uacc = {};
    f32x16 oa = oacc[ib];
#pragma unroll
    for (int kb = 0; kb <= ib; ++kb) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int col = kb * 32 + c * 16 + half * 4;
        u16x8 frag[2][2];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int hl = 0; hl < 2; ++hl) {
            const u16x4 x0 = *reinterpret_cast<const u16x4*>(&sm.stage[m][hl][l32][col]);
            const u16x4 x1 = *reinterpret_cast<const u16x4*>(&sm.stage[m][hl][l32][col + 8]);
            frag[m][hl] = (u16x8){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          }
        const bf16x8 rhi = Rb[kb][c][0], rlo = Rb[kb][c][1];
        uacc = mfma32(as_bf16x8(frag[0][0]), rhi, uacc);
        uacc = mfma32(as_bf16x8(frag[0][0]), rlo, uacc);
        uacc = mfma32(as_bf16x8(frag[0][1]), rhi, uacc);
        oa = mfma32(as_bf16x8(frag[1][0]), rhi, oa);
        oa = mfma32(as_bf16x8(frag[1][0]), rlo, oa);
        oa = mfma32(as_bf16x8(frag[1][1]), rhi, oa);
      }
    }
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const int i = ib * 32 + 8 * (rr >> 2) + 4 * half + (rr & 3);
      if (i < n) {
        const size_t off = ((size_t)(ns + i) * a.H + h) * D + vcol;
        a.u[off] = uacc[rr];
        a.o[off] = oa[rr];
      }
    }
  }
}

template <int NT>
int launch_gdn(const GdnArgs& args, hipStream_t stream) {
  const int G = args.H / args.HK;
  const int P = args.R * args.HK;
  const int P8 = (P + 7) / 8;
  const dim3 grid(8 * P8 * G);
  hipLaunchKernelGGL(tree_gdn_kernel<NT>, grid, dim3(NTHREADS), 0, stream, args);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

}  // namespace

extern "C" int mfd_tree_gdn(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum,
                            const float* beta, const float* s0, const int32_t* parents, const int8_t* anc8,
                            const int32_t* cu_nodes, int R, int N, int HK, int H, int D_, int max_nodes, float* u,
                            float* o, int32_t* err_flag, void* stream) {
  if (D_ != D) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_tree_gdn: head dim %d (only %d)", D_, D);
  if (R < 1 || N < 0 || HK < 1 || H < 1 || H % HK != 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gdn: bad sizes R=%d N=%d HK=%d H=%d", R, N, HK, H);
  if (!cu_nodes && R != 1) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gdn: cu_nodes required for R > 1");
  if (!parents && (!anc8 || R != 1))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gdn: parents required unless R == 1 and anc8 given");
  if (max_nodes < 0 || max_nodes > MFD_GDN_MAX_NODES)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_tree_gdn: max_nodes %d exceeds %d", max_nodes, MFD_GDN_MAX_NODES);
  if (!cu_nodes && N > max_nodes)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gdn: N=%d > max_nodes=%d", N, max_nodes);
  if (N == 0 || max_nodes == 0) return MFD_OK;
  if (!q || !k || !v || !g_cum || !beta || !s0 || !u || !o)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gdn: null tensor pointer");
  GdnArgs args{q, k, v, g_cum, beta, s0, parents, anc8, cu_nodes, u, o, err_flag, R, N, HK, H};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (max_nodes <= 32) return launch_gdn<1>(args, s);
  if (max_nodes <= 64) return launch_gdn<2>(args, s);
  return launch_gdn<4>(args, s);
}
