// Tree gated-delta-rule verification of trees above 128 nodes (up to MFD_GDN_MAX_NODES), gfx950.
//
// Same quantities as the fused kernel (tree_gdn.hip; inference/hf/tree_gdn_kernel.py:3-6,
// inference/hf/qwen35_tree.py:9-20): for the nodes of one tree in topological order,
//   u = (I + A)^{-1} R,  R_i = beta_i (v_i - e^{G_i} S0^T k_i),   A_ij = beta_i e^{G_i-G_j} k_i.k_j (strict anc.)
//   o = E + P u,         E_i = e^{G_i} S0^T q_i,                  P_ij = e^{G_i-G_j} q_i.k_j   (anc. or self)
// The fused kernel holds a whole tree's K / Q / v rows in LDS, which a 512-node tree does not fit. Here every
// quantity is kept per root-path slot (a node has at most MAXD ancestors-or-self), so the work and the LDS
// footprint grow linearly in the node count:
//   tree_ctx_large_kernel   one workgroup per request: each node's root path (node ids by depth) and depth
//   tree_gram_kernel        one workgroup per (request, key head, 32-node chunk): the Gram entries k_i.k_j and
//                           q_i.k_j of the chunk's nodes against their ancestors (MFMA over the 32 x 32 blocks
//                           that hold an ancestor pair), written per path slot: gram[node][key head][2][MAXD]
//   tree_gdn_large_kernel   one workgroup per (request, value head, 32 value columns):
//     A  a_i[s] = beta_i e^{G_i-G_j} kk_i[s] (strict), p_i[s] = e^{G_i-G_j} qk_i[s], j = path_i[s]
//     T  rows of T = (I + A)^{-1} by path-local back substitution (one thread per node)
//     W  rows of W = P T
//     R  per 16-node tile: K S0 and Q S0 on MFMA (S0 split into bf16 hi + lo, so fp32-accurate):
//        R = beta (v - e^G K S0) into LDS, E = e^G Q S0 kept in registers
//     O  u_i = sum_s T_i[s] R_{path_i[s]},  o_i = E_i + sum_s W_i[s] R_{path_i[s]}  (fp32, <= MAXD terms)
// The sub-units of one (request, key head) sit on one XCD, so its q / k rows and Gram rows are read from
// HBM once and from that XCD's L2 after.
#include "gdn_common.h"

namespace {
using namespace gdn;

constexpr int CG = 32;        // value columns per workgroup of the main kernel
constexpr int NCG = D / CG;   // column groups per value head

// Tree context of one request for the large-tree path (global memory; one block per request).
template <int NMAX>
struct alignas(16) TreeMetaL {
  uint16_t path[NMAX][MAXD];  // path[i][s] = ancestor of i at depth s + 1 for s < depth[i] (path[i][depth-1] = i);
                              // i for s >= depth[i]; 0 for i >= n
  uint8_t depth[NMAX];        // nodes on the root path of i (0 for i >= n)
  int32_t bad;                // MFD_DEVERR_* bits of the tree
  int32_t n;                  // nodes of the request
  int32_t nmax;               // NMAX of the layout
  int32_t pad;
};
static_assert(sizeof(TreeMetaL<256>) % 16 == 0 && sizeof(TreeMetaL<512>) % 16 == 0, "16-byte copies");
template <int NMAX>
constexpr uint32_t meta_depth_off() { return (uint32_t)(NMAX * MAXD * 2); }

template <int NMAX>
__global__ __launch_bounds__(NMAX) void tree_ctx_large_kernel(const int32_t* parents, const int8_t* anc8,
                                                              const int32_t* cu_nodes, int N, uint8_t* ctx,
                                                              int32_t* err) {
  __shared__ TreeMetaL<NMAX> m;
  __shared__ int par[NMAX];
  const int tid = threadIdx.x;
  const int r = blockIdx.x;
  int ns, n;
  request_range(cu_nodes, r, N, ns, n);
  const bool fits = n <= NMAX;
  if (tid == 0) {
    m.bad = fits ? 0 : MFD_DEVERR_TOO_MANY_NODES;
    m.n = n;
    m.nmax = NMAX;
    m.pad = 0;
  }
  const int live = fits && tid < n;
  par[tid] = live ? parent_of(parents, anc8, ns, tid, n) : -1;
  __syncthreads();
  // walk up the parents; the chain stays in registers
  int d = 0;
  int chain[MAXD + 1];
  if (live) {
    int cur = tid;
#pragma unroll
    for (int s = 0; s <= MAXD; ++s) {
      chain[s] = cur;
      if (cur >= 0) {
        const int p = par[cur];
        if (p >= cur || p < -1) {
          atomicOr(&m.bad, MFD_DEVERR_NOT_TOPOLOGICAL);
          cur = -1;
        } else {
          cur = p;
        }
        ++d;
      }
    }
    if (cur >= 0 || d > MAXD) {
      atomicOr(&m.bad, MFD_DEVERR_TOO_DEEP);
      d = 0;
    }
  }
  const uint16_t self = (uint16_t)(live ? tid : 0);
#pragma unroll
  for (int s = 0; s < MAXD; ++s) m.path[tid][s] = self;
#pragma unroll
  for (int s = 0; s < MAXD; ++s)
    if (s < d) m.path[tid][d - 1 - s] = (uint16_t)chain[s];
  m.depth[tid] = (uint8_t)d;
  __syncthreads();
  if (tid == 0 && m.bad && err) atomicOr(err, m.bad);
  constexpr int NCM = (int)(sizeof(TreeMetaL<NMAX>) / 16);
  const uint4* src = reinterpret_cast<const uint4*>(&m);
  uint4* dst = reinterpret_cast<uint4*>(ctx + (size_t)r * sizeof(TreeMetaL<NMAX>));
  for (int c = tid; c < NCM; c += NMAX) dst[c] = src[c];
}

__device__ __forceinline__ bf16x8 ldg8(const uint16_t* p) { return as_bf16x8(*reinterpret_cast<const u16x8*>(p)); }

// Gram entries of 32 nodes (chunk T of request r) against their ancestors, for key head hk.
template <int NMAX>
__global__ __launch_bounds__(256) void tree_gram_kernel(GdnLargeArgs a) {
  const int T = blockIdx.x;
  const int r = blockIdx.y / a.HK;
  const int hk = blockIdx.y % a.HK;
  int ns, n;
  request_range(a.cu_nodes, r, a.N, ns, n);
  if (32 * T >= n || n > NMAX) return;
  const TreeMetaL<NMAX>* m = reinterpret_cast<const TreeMetaL<NMAX>*>(a.ctx) + r;
  if (m->bad != 0 || m->n != n || m->nmax != NMAX) return;  // rejected: the main kernel reports it

  __shared__ float kk[32][MAXD + 1], qk[32][MAXD + 1];
  __shared__ uint16_t pth[32][MAXD];
  __shared__ int dep[32];
  __shared__ uint32_t jmask;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i0 = 32 * T;
  for (int x = tid; x < 32 * MAXD; x += 256) {
    const int row = x / MAXD, s = x % MAXD;
    pth[row][s] = m->path[i0 + row][s];
    kk[row][s] = 0.f;
    qk[row][s] = 0.f;
  }
  if (tid < 32) dep[tid] = (i0 + tid < n) ? m->depth[i0 + tid] : 0;
  if (tid == 0) jmask = 0u;
  __syncthreads();
  // chunks that hold an ancestor of some row (the chunk itself always does)
  for (int x = tid; x < 32 * MAXD; x += 256) {
    const int row = x / MAXD, s = x % MAXD;
    if (s < dep[row]) atomicOr(&jmask, 1u << (pth[row][s] >> 5));
  }
  __syncthreads();
  const uint32_t jm = jmask;

  // fragments of 32x32x16: lane l holds row l % 32 and k = 16 ks + 8 (l / 32) .. + 7
  const int g2 = lane >> 5, l32 = lane & 31;
  const int HKD = a.HK * D;
  const uint16_t* kb = a.k + (size_t)ns * HKD + hk * D;
  const uint16_t* qb = a.q + (size_t)ns * HKD + hk * D;
  const int ri = min(i0 + l32, n - 1);
  bf16x8 fa[D / 16], fq[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    fa[ks] = ldg8(kb + (size_t)ri * HKD + 16 * ks + 8 * g2);
    fq[ks] = ldg8(qb + (size_t)ri * HKD + 16 * ks + 8 * g2);
  }
  int cnt = 0;
  for (int J = 0; J <= T; ++J) {
    if (!((jm >> J) & 1u)) continue;
    if ((cnt++ & 3) != w) continue;
    const int j = 32 * J + l32;
    const int rj = min(j, n - 1);
    f32x16 gkk = {}, gqk = {};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const bf16x8 bk = ldg8(kb + (size_t)rj * HKD + 16 * ks + 8 * g2);
      gkk = mfma32(fa[ks], bk, gkk);
      gqk = mfma32(fq[ks], bk, gqk);
    }
    // C register x: row 8 (x / 4) + 4 g2 + x % 4, column j. j is on row i's root path iff path_i[depth_j - 1] == j.
    const int sj = (j < n) ? (int)m->depth[j] - 1 : -1;
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int row = 8 * (x >> 2) + 4 * g2 + (x & 3);
      if (sj >= 0 && sj < dep[row] && pth[row][sj] == j) {
        qk[row][sj] = gqk[x];
        if (j != i0 + row) kk[row][sj] = gkk[x];
      }
    }
  }
  __syncthreads();
  float* gb = a.gram + ((size_t)ns * a.HK + hk) * (2 * MAXD);
  for (int x = tid; x < 32 * 2 * MAXD; x += 256) {
    const int row = x / (2 * MAXD), e = x % (2 * MAXD);
    if (i0 + row < n) gb[(size_t)(i0 + row) * a.HK * (2 * MAXD) + e] = e < MAXD ? kk[row][e] : qk[row][e - MAXD];
  }
}

template <int NMAX>
struct alignas(16) LargeSmem {
  union {
    float kq[NMAX][2 * MAXD];  // Gram row of node i (k.k slots, then q.k slots); phase A turns k.k into a_i
    float R[NMAX][CG];         // phases R - O: the R rows of this workgroup's value columns
  };
  float T[NMAX][MAXD];         // T_i[s] (0 past the depth)
  float W[NMAX][MAXD];         // W_i[s] (0 past the depth)
  uint16_t path[NMAX][MAXD];
  uint8_t depth[NMAX];
  float G[NMAX], beta[NMAX], eG[NMAX];
};

template <int NMAX>
constexpr int large_threads() { return NMAX < 256 ? 256 : NMAX; }

template <int NMAX>
__global__ __launch_bounds__(large_threads<NMAX>()) void tree_gdn_large_kernel(GdnLargeArgs a) {
  constexpr int NT = large_threads<NMAX>();
  constexpr int NW = NT / 64;
  constexpr int NTG = NW / 2;                              // waves per 16-column tile
  constexpr int MAXT = (NMAX / 16 + NTG - 1) / NTG;        // 16-node tiles per wave
  __shared__ LargeSmem<NMAX> sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4;
  const int l16 = lane & 15;

  // workgroup -> (request, key head, value head member x column group); the sub-units of one
  // (request, key head) land on one XCD (workgroup id modulo 8)
  const int Gq = a.H / a.HK;
  const int SUB = Gq * NCG;
  const int P = a.R * a.HK;
  const int id = blockIdx.x;
  const int rest = id >> 3;
  const int pidx = (rest / SUB) * 8 + (id & 7);
  if (pidx >= P) return;
  const int sub = rest % SUB;
  const int r = pidx / a.HK;
  const int hk = pidx % a.HK;
  const int h = hk * Gq + sub / NCG;
  const int cg = sub % NCG;
  int ns, n;
  request_range(a.cu_nodes, r, a.N, ns, n);
  ns = __builtin_amdgcn_readfirstlane(ns);
  n = __builtin_amdgcn_readfirstlane(n);
  if (n <= 0) return;
  const TreeMetaL<NMAX>* m = reinterpret_cast<const TreeMetaL<NMAX>*>(a.ctx) + r;
  const int rej = (n > NMAX) ? MFD_DEVERR_TOO_MANY_NODES
                             : (m->bad | ((m->n != n || m->nmax != NMAX) ? MFD_DEVERR_BAD_CONTEXT : 0));
  if (rej) {
    nan_fill(a.u, a.o, ns, n, a.H, h, cg * CG, CG, tid, NT);
    if (tid == 0 && a.err) atomicOr(a.err, rej);
    return;
  }
  const int HD = a.H * D, HKD = a.HK * D;
  const int nt16 = (n + 15) >> 4;

  // ---- phase 0: this lane's S0 column (registers); gates; root paths, depths and Gram rows straight into LDS.
  //      Everything is waited for before the tree phases (vmcnt(0): the direct-to-LDS loads are not tracked
  //      by the compiler); the first tile's q / k rows are requested right after, in flight through them.
  const int ct = w & 1;           // 16-column tile of this wave
  const int tg = w >> 1;          // tile group of this wave
  const int vcol = cg * CG + ct * 16 + l16;
  const __amdgpu_buffer_rsrc_t rs_s0 = rsrc(a.s0 + ((size_t)r * a.H + h) * D * D, D * D * 4);
  float raw[D / 32][8];
  {
    const uint32_t voff = (uint32_t)(g4 * 8 * D + vcol) * 4u;
#pragma unroll
    for (int c = 0; c < D / 32; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        raw[c][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_s0, voff, (c * 32 + e) * D * 4, 2));
  }
  {
    float g = 0.f, b = 0.f;
    if (tid < n) {
      g = a.g_cum[(size_t)(ns + tid) * a.H + h];
      b = a.beta[(size_t)(ns + tid) * a.H + h];
    }
    const int np = 2 * n, nd = (n + 15) >> 4, ngr = 8 * n;
    for (int c0 = w * 64; c0 < np; c0 += NT)
      if (c0 + lane < np) dma16_s(m, (uint32_t)(c0 + lane) * 16u, lds_addr(&sm.path[0][0]) + (uint32_t)c0 * 16u);
    for (int c0 = w * 64; c0 < nd; c0 += NT)
      if (c0 + lane < nd)
        dma16_s(m, meta_depth_off<NMAX>() + (uint32_t)(c0 + lane) * 16u, lds_addr(&sm.depth[0]) + (uint32_t)c0 * 16u);
    const float* gb = a.gram + ((size_t)ns * a.HK + hk) * (2 * MAXD);
    for (int c0 = w * 64; c0 < ngr; c0 += NT) {
      const int c = c0 + lane;
      if (c < ngr)
        dma16_s(gb, (uint32_t)((c >> 3) * a.HK * (2 * MAXD) + (c & 7) * 4) * 4u,
                lds_addr(&sm.kq[0][0]) + (uint32_t)c0 * 16u);
    }
    if (tid < NMAX) {
      sm.G[tid] = g;
      sm.beta[tid] = b;
      sm.eG[tid] = __expf(g);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();
  const uint16_t* kb = a.k + (size_t)ns * HKD + hk * D + 8 * g4;
  const uint16_t* qb = a.q + (size_t)ns * HKD + hk * D + 8 * g4;
  bf16x8 fk[D / 32], fq[D / 32];
  auto load_frags = [&](int t) __attribute__((always_inline)) {
    const int rc = min(16 * t + l16, n - 1);
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      fk[c] = ldg8(kb + (size_t)rc * HKD + 32 * c);
      fq[c] = ldg8(qb + (size_t)rc * HKD + 32 * c);
    }
  };
  if (tg < nt16) load_frags(tg);

  // ---- phase A: a_i (strict ancestors, in place over k.k) and p_i (registers) of node i = tid
  float preg[MAXD];
  const int i_me = tid < n ? tid : 0;
  const int d_me = tid < n ? (int)sm.depth[i_me] : 0;
  int pth[MAXD];
#pragma unroll
  for (int s = 0; s < MAXD; ++s) pth[s] = sm.path[i_me][s];
  if (tid < n) {
    const float gi = sm.G[i_me];
    const float bi = sm.beta[i_me];
#pragma unroll
    for (int s4 = 0; s4 < MAXD; s4 += 4) {
      f32x4 xa = *reinterpret_cast<const f32x4*>(&sm.kq[i_me][s4]);
      const f32x4 xp = *reinterpret_cast<const f32x4*>(&sm.kq[i_me][MAXD + s4]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int s = s4 + e;
        const float ex = __expf(gi - sm.G[pth[s]]);
        xa[e] = (s < d_me - 1) ? xa[e] * (bi * ex) : 0.f;
        preg[s] = (s < d_me) ? xp[e] * ex : 0.f;
      }
      *reinterpret_cast<f32x4*>(&sm.kq[i_me][s4]) = xa;
    }
  }
  __syncthreads();
  // ---- phase T: T_i[d-1] = 1, T_i[s] = -sum_{m>s} T_i[m] a_{path(m)}[s] (right-looking over m)
  if (tid < n) {
    float acc[MAXD], Tr[MAXD];
#pragma unroll
    for (int s = 0; s < MAXD; ++s) acc[s] = 0.f;
#pragma unroll
    for (int mm = MAXD - 1; mm >= 0; --mm) {
      const float tm = (mm < d_me) ? ((mm == d_me - 1) ? 1.f : -acc[mm]) : 0.f;
      Tr[mm] = tm;
      if (mm > 0) {
        const int j = pth[mm];
#pragma unroll
        for (int s4 = 0; s4 < mm; s4 += 4) {
          const f32x4 row = *reinterpret_cast<const f32x4*>(&sm.kq[j][s4]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (s4 + e < mm) acc[s4 + e] = fmaf(tm, row[e], acc[s4 + e]);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < MAXD; s += 4)
      *reinterpret_cast<f32x4*>(&sm.T[i_me][s]) = (f32x4){Tr[s], Tr[s + 1], Tr[s + 2], Tr[s + 3]};
  }
  __syncthreads();  // T rows complete; the Gram rows are dead from here on (R overwrites them)
  // ---- phase W: W_i[s] = sum_{m>=s} p_i[m] T_{path(m)}[s]
  if (tid < n) {
    float Wr[MAXD];
#pragma unroll
    for (int s = 0; s < MAXD; ++s) Wr[s] = 0.f;
#pragma unroll
    for (int mm = 0; mm < MAXD; ++mm) {
      const int j = pth[mm];
#pragma unroll
      for (int s4 = 0; s4 <= mm; s4 += 4) {
        const f32x4 row = *reinterpret_cast<const f32x4*>(&sm.T[j][s4]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (s4 + e <= mm) Wr[s4 + e] = fmaf(preg[mm], row[e], Wr[s4 + e]);
      }
    }
#pragma unroll
    for (int s = 0; s < MAXD; s += 4)
      *reinterpret_cast<f32x4*>(&sm.W[i_me][s]) = (f32x4){Wr[s], Wr[s + 1], Wr[s + 2], Wr[s + 3]};
  }

  // ---- phase R: per 16-node tile t of this wave: K S0 -> R (LDS), Q S0 -> E (registers); S0 as bf16 hi + lo
  bf16x8 sh[D / 32], sl[D / 32];
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    u32x4 hv, lv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t h2, l2;
      split2_bf16(raw[c][2 * e], raw[c][2 * e + 1], h2, l2);
      hv[e] = h2;
      lv[e] = l2;
    }
    sh[c] = __builtin_bit_cast(bf16x8, hv);
    sl[c] = __builtin_bit_cast(bf16x8, lv);
  }
  const uint16_t* vb = a.v + (size_t)ns * HD + h * D + vcol;
  f32x4 E[MAXT];
#pragma unroll
  for (int tt = 0; tt < MAXT; ++tt) {
    const int t = tg + tt * NTG;
    E[tt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (t < nt16) {
      float vv[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) vv[rr] = bf2f(vb[(size_t)min(16 * t + 4 * g4 + rr, n - 1) * HD]);
      f32x4 ak = {0.f, 0.f, 0.f, 0.f}, akl = ak, eq = ak, eql = ak;
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        ak = mfma16(fk[c], sh[c], ak);
        akl = mfma16(fk[c], sl[c], akl);
        eq = mfma16(fq[c], sh[c], eq);
        eql = mfma16(fq[c], sl[c], eql);
      }
      if (t + NTG < nt16) load_frags(t + NTG);
      ak += akl;
      eq += eql;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = 16 * t + 4 * g4 + rr;
        sm.R[i][ct * 16 + l16] = sm.beta[i] * (vv[rr] - sm.eG[i] * ak[rr]);
        E[tt][rr] = sm.eG[i] * eq[rr];
      }
    }
  }
  __syncthreads();  // R and W rows complete

  // ---- phase O: u_i = sum_s T_i[s] R_{path_i[s]}, o_i = E_i + sum_s W_i[s] R_{path_i[s]}
  float* ub = a.u + (size_t)ns * HD + h * D + vcol;
  float* ob = a.o + (size_t)ns * HD + h * D + vcol;
  const int col = ct * 16 + l16;
#pragma unroll
  for (int tt = 0; tt < MAXT; ++tt) {
    const int t = tg + tt * NTG;
    if (t >= nt16) break;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int i = 16 * t + 4 * g4 + rr;
      const bool live = i < n;
      const int ic = live ? i : n - 1;
      const int d = live ? (int)sm.depth[ic] : 0;
      float uacc = 0.f, oacc = E[tt][rr];
      for (int sb = 0; sb < MAXD / 4; ++sb) {
        if (__builtin_amdgcn_ballot_w64(4 * sb < d) == 0) break;
        const u32x2 pp = *reinterpret_cast<const u32x2*>(&sm.path[ic][4 * sb]);
        const f32x4 tv = *reinterpret_cast<const f32x4*>(&sm.T[ic][4 * sb]);
        const f32x4 wv = *reinterpret_cast<const f32x4*>(&sm.W[ic][4 * sb]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = (int)((pp[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
          const float rv = sm.R[j][col];
          uacc = fmaf(tv[e], rv, uacc);
          oacc = fmaf(wv[e], rv, oacc);
        }
      }
      if (live) {
        ub[(size_t)i * HD] = uacc;
        ob[(size_t)i * HD] = oacc;
      }
    }
  }
}

template <int NMAX>
int run_large(const GdnLargeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(tree_gram_kernel<NMAX>, dim3(NMAX / 32, a.R * a.HK), dim3(256), 0, s, a);
  MFD_CHECK_LAUNCH();
  const int P = a.R * a.HK;
  const int SUB = (a.H / a.HK) * NCG;
  const dim3 grid(8 * ((P + 7) / 8) * SUB);
  hipLaunchKernelGGL(tree_gdn_large_kernel<NMAX>, grid, dim3(large_threads<NMAX>()), 0, s, a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

}  // namespace

size_t gdn_large_ctx_block_bytes(int max_nodes) {
  return max_nodes <= 256 ? sizeof(TreeMetaL<256>) : sizeof(TreeMetaL<512>);
}

int gdn_large_context(const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R, int N,
                      int max_nodes, uint8_t* ctx, int32_t* err, hipStream_t s) {
  if (max_nodes <= 256)
    hipLaunchKernelGGL(tree_ctx_large_kernel<256>, dim3(R), dim3(256), 0, s, parents, anc8, cu_nodes, N, ctx, err);
  else
    hipLaunchKernelGGL(tree_ctx_large_kernel<512>, dim3(R), dim3(512), 0, s, parents, anc8, cu_nodes, N, ctx, err);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

int gdn_large_run(const GdnLargeArgs& a, int max_nodes, hipStream_t s) {
  return max_nodes <= 256 ? run_large<256>(a, s) : run_large<512>(a, s);
}
