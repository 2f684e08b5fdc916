// Exact mixture-tree builder for gfx950: one wave per request runs the best-first expansion of the
// reference's C++ heap (inference/hf/tree_build_ext.py:48-62 MixEntry / MixGreater, :158-203 build_mixture;
// batched form inference/sglang/patches/sglang-v0.5.22-mfd.patch:1330-1407) node for node:
//   - key = -(float(logw) + prior[mode]) in fp32, logw accumulated in fp64 as (logw - lp[r]) + lp[r + 1]
//     for a sibling and logw + lp[d][0] for a child;
//   - pop order: key, then mode, parent, depth, rank ascending (entries are unique in (mode, parent, rank),
//     so the logw tie-break of the reference is never reached): an entry's order is the pair
//     (order-preserving bits of the fp32 key, fields = mode 4b | parent 12b | depth 6b | rank 10b);
//   - a prefix popped again by another mode reuses its node (lookup by (parent, token)); the budget
//     counts distinct nodes.
// The frontier lives in LDS; slot s belongs to lane s % 64, and every lane keeps the best of its own
// slots in registers. A pop is one wave minimum over those 64 candidates: the fp32 key bits through
// DPP row rotations and four lane reads (the fields only when two lanes tie on the key). The popped
// slot is reused by its sibling (its lane rescans its slots), the child takes the next slot (its lane
// compares it with its best). The node table (parent, token of nodes 1..budget) is held in registers,
// node j + 1 by lane j % 64, so the (parent, token) lookup is one compare and a ballot. The request's top
// log-probs / ids are staged in LDS.
// Outputs: tree[b] = tokens, depths, parents of width budget + 1 (index 0 = root: token 0, depth 0,
// parent -1; tail entries 0, 0, -1), counts[b], and optionally the ancestor-or-self matrix anc8[b]
// ([budget + 1]^2 int8, row i = row of parent(i) plus i; inference/hf/tree_build_ext.py:101-110).
#include "mfd_common.h"

namespace {

constexpr int WAVE = 64;
constexpr uint32_t NONE = 0xFFFFFFFFu;  // key bits / fields of a dead slot (orders after every live entry)

struct BuildArgs {
  const float* lp;       // [bs, K, L, k]
  const void* ids;       // [bs, K, L, k] int32 or int64
  int ids_int64;
  const float* prior;    // [bs, K] or null (zeros)
  int bs, K, L, k, budget, cap;
  int64_t* tree;         // [bs, 3, budget + 1]
  int64_t* counts;       // [bs]
  int8_t* anc8;          // [bs, budget + 1, budget + 1] or null
  int32_t* err;
};

__device__ __forceinline__ uint32_t umin32(uint32_t x, uint32_t y) { return x < y ? x : y; }
// DPP row rotation by N lanes within each row of 16 (every source lane exists, so no bound control)
template <int N>
__device__ __forceinline__ uint32_t row_ror(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + N, 0xF, 0xF, false);
}
// minimum over the 64 lanes, returned wave-uniform: rotations 1, 2, 4, 8 leave every lane of a row
// with the row minimum, then the four row minima are read into scalar registers
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = umin32(v, row_ror<1>(v));
  v = umin32(v, row_ror<2>(v));
  v = umin32(v, row_ror<4>(v));
  v = umin32(v, row_ror<8>(v));
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return umin32(umin32(r0, r1), umin32(r2, r3));
}
__device__ __forceinline__ uint32_t pack_fields(int mode, int parent, int depth, int rank) {
  return ((uint32_t)mode << 28) | ((uint32_t)parent << 16) | ((uint32_t)depth << 10) | (uint32_t)rank;
}
__device__ __forceinline__ uint32_t key_bits(float key) { return float_order_key(key + 0.0f); }
// dst[i] = (int32) src[i] for i < n, by one wave: batches of 16 loads per lane, issued before any is used
template <typename T>
__device__ __forceinline__ void stage_lds(const T* src, int32_t* dst, int n, int lane) {
  constexpr int SB = 16;
  for (int i0 = 0; i0 < n; i0 += SB * WAVE) {
    int32_t v[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) v[u] = (int32_t)src[min(i0 + u * WAVE + lane, n - 1)];
#pragma unroll
    for (int u = 0; u < SB; ++u)
      if (i0 + u * WAVE + lane < n) dst[i0 + u * WAVE + lane] = v[u];
  }
}

// Outputs of request b: tree[b] = tokens, depths, parents of width budget + 1 (index 0 = root; tail entries
// 0, 0, -1), counts[b], and the ancestor-or-self matrix when requested.
__device__ void write_tree(const BuildArgs& a, int b, int lane, int count, const int32_t* npar, const int32_t* ntok,
                           const int32_t* ndep) {
  const int W = a.budget + 1;
  int64_t* t = a.tree + (int64_t)b * 3 * W;
  for (int i = lane; i < W; i += WAVE) {
    const bool used = i <= count;
    t[i] = (used && i > 0) ? (int64_t)ntok[i] : 0;
    t[W + i] = used ? (int64_t)ndep[i] : 0;
    t[2 * W + i] = used ? (int64_t)npar[i] : -1;
  }
  if (lane == 0) a.counts[b] = count;
  if (a.anc8) {
    int8_t* vis = a.anc8 + (int64_t)b * W * W;
    // zero the matrix with wave-coalesced stores, make those stores visible to the wave, then set the
    // ancestor-or-self entries of rows 0..count (one row per lane, walking up the parents)
    const int64_t WW = (int64_t)W * W;
    // bytes up to the first 16-byte boundary, 16-byte stores, then the remaining bytes
    const int64_t head = min(WW, (int64_t)((16 - (reinterpret_cast<uintptr_t>(vis) & 15)) & 15));
    const int64_t nvec = (WW - head) / 16;
    for (int64_t f = lane; f < head; f += WAVE) vis[f] = 0;
    uint4* vv = reinterpret_cast<uint4*>(vis + head);
    for (int64_t f = lane; f < nvec; f += WAVE) vv[f] = make_uint4(0u, 0u, 0u, 0u);
    for (int64_t f = head + nvec * 16 + lane; f < WW; f += WAVE) vis[f] = 0;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i <= count; i += WAVE) {
      int8_t* row = vis + (int64_t)i * W;
      int cur = i;
      while (cur >= 0) {
        row[cur] = 1;
        cur = npar[cur];
      }
    }
  }
}

// (token, log-prob bits) records of the request's top lists, staged by one wave: batches of 16 entries per
// lane, all loads issued before the first one is used (int64 ids keep their low 32 bits)
template <typename T>
__device__ __forceinline__ void stage_records(const float* lp, const T* ids, int2* rec, int n, int lane) {
  constexpr int SB = 16;
  for (int i0 = 0; i0 < n; i0 += SB * WAVE) {
    float v[SB];
    int32_t t[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int i = min(i0 + u * WAVE + lane, n - 1);
      v[u] = lp[i];
      t[u] = (int32_t)ids[i];
    }
#pragma unroll
    for (int u = 0; u < SB; ++u)
      if (i0 + u * WAVE + lane < n) rec[i0 + u * WAVE + lane] = make_int2(t[u], __float_as_int(v[u]));
  }
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)u, l), hi = __builtin_amdgcn_readlane((uint32_t)(u >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Frontier rows held in registers: slot s belongs to lane s % 64, row s / 64; rows below RR are registers,
// rows from RR on (large or heavily merged frontiers) live in LDS.
constexpr int RR = 2;

// LDS layout (dynamic): frontier rows >= RR: logw f64 [cap], key bits u32 [cap], fields u32 [cap] (indexed by
// slot), records (token, lp bits) [K L k], prior f32 [16], node parent / token / depth i32 [budget + 1]
// (filled from the register node table at the end).
// NR = register slots per lane of the node table (64 NR >= budget).
//
// A pop needs no LDS round trip: every lane keeps its best slot's key, fields, row and logw in registers, and
// after each pop every lane prefetches the records its best entry will need if popped (token and log-prob
// of its rank, the log-prob of the next rank, the first log-prob of the next depth, the mode's prior); the
// prefetch lands while the next wave minimum is computed. Replacing the popped slot by its sibling and
// rescanning the winner's register rows, and comparing the child with the best of its lane, are register
// operations.
template <int NR>
__global__ __launch_bounds__(WAVE) void build_mixture_kernel(BuildArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char smem[];
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int K = a.K, L = a.L, kk = a.k, cap = a.cap, budget = a.budget;
  const int nlp = K * L * kk;
  double* flogw = reinterpret_cast<double*>(smem);
  uint32_t* fhi = reinterpret_cast<uint32_t*>(flogw + cap);
  uint32_t* flo = fhi + cap;
  int2* rec = reinterpret_cast<int2*>(flo + cap);
  float* sprior = reinterpret_cast<float*>(rec + nlp);
  int32_t* npar = reinterpret_cast<int32_t*>(sprior + 16);
  int32_t* ntok = npar + (budget + 1);
  int32_t* ndep = ntok + (budget + 1);

  const float* lpb = a.lp + (int64_t)b * nlp;
  if (a.ids_int64)
    stage_records(lpb, static_cast<const int64_t*>(a.ids) + (int64_t)b * nlp, rec, nlp, lane);
  else
    stage_records(lpb, static_cast<const int32_t*>(a.ids) + (int64_t)b * nlp, rec, nlp, lane);

  // register frontier rows; unused slots hold NONE keys and never win
  uint32_t khi[RR], klo[RR];
  double klw[RR];
#pragma unroll
  for (int rr = 0; rr < RR; ++rr) {
    khi[rr] = NONE;
    klo[rr] = NONE;
    klw[rr] = 0.0;
  }
  // this lane's best live slot: key bits, fields, row, logw
  uint32_t lhi = NONE, llo = NONE;
  int lrow = 0;
  double lbw = 0.0;
  // seed: one entry per mode (rank 0 at depth 1 under the root) in slot m, which lane m owns (K <= 16)
  if (lane < K) {
    const float pr = a.prior ? a.prior[(int64_t)b * K + lane] : 0.f;
    sprior[lane] = pr;
    const double lw = (double)lpb[(int64_t)lane * L * kk];
    lhi = key_bits(-((float)lw + pr));
    llo = pack_fields(lane, 0, 1, 0);
    khi[0] = lhi;
    klo[0] = llo;
    klw[0] = lw;
    lbw = lw;
  }
  int32_t rpar[NR], rtok[NR], rdep[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    rpar[r] = -1;  // never equals a parent id
    rtok[r] = 0;
    rdep[r] = 0;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();

  // records of this lane's best entry (mode m, depth d, rank r): token and lp of (m, d, r), lp of rank r + 1,
  // lp of (m, d + 1, 0), prior of m. Lanes without a live slot read entry 0.
  int ptok;
  float plp, plp1, plpc, ppr;
  auto prefetch = [&]() __attribute__((always_inline)) {
    const bool live = lhi != NONE;
    const int m = live ? (int)(llo >> 28) : 0;
    const int dm1 = live ? (int)((llo >> 10) & 0x3F) - 1 : 0;
    const int r = live ? (int)(llo & 0x3FF) : 0;
    const int row0 = (m * L + dm1) * kk;
    const int2 e = rec[row0 + r];
    ptok = e.x;
    plp = __int_as_float(e.y);
    plp1 = __int_as_float(rec[row0 + min(r + 1, kk - 1)].y);
    plpc = __int_as_float(rec[(m * L + min(dm1 + 1, L - 1)) * kk].y);
    ppr = sprior[m];
  };
  prefetch();

  int count = 0, tail = K, alive = K;
  bool overflow = false;
  // every iteration consumes a frontier entry and at most cap entries are ever pushed: bounded loop
  for (int iter = 0; iter < cap && alive > 0 && count < budget; ++iter) {
    // ---- pop: the lane holding the smallest (key bits, fields)
    const uint32_t mh = wave_min_u32(lhi);
    const uint64_t tie = __builtin_amdgcn_ballot_w64(lhi == mh);
    int win = (int)__builtin_ctzll(tie);
    if (__builtin_popcountll(tie) > 1) {
      const uint32_t ml = wave_min_u32(lhi == mh ? llo : NONE);
      win = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(lhi == mh && llo == ml));
    }
    const uint32_t f = __builtin_amdgcn_readlane(llo, win);
    const int row = __builtin_amdgcn_readlane(lrow, win);
    const double logw = readlane_f64(lbw, win);
    const int token = __builtin_amdgcn_readlane(ptok, win);
    const float lp_r = readlane_f32(plp, win);
    const float lp_r1 = readlane_f32(plp1, win);
    const float lp_c = readlane_f32(plpc, win);
    const float pr = readlane_f32(ppr, win);
    const int mode = (int)(f >> 28);
    const int parent = (int)((f >> 16) & 0xFFF);
    const int depth = (int)((f >> 10) & 0x3F);
    const int rank = (int)(f & 0x3FF);
    // ---- node of (parent, token), or a new node
    int current = 0;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint64_t h = __builtin_amdgcn_ballot_w64(rpar[r] == parent && rtok[r] == token);
      if (h != 0 && current == 0) current = 64 * r + (int)__builtin_ctzll(h) + 1;
    }
    if (current == 0) {
      current = ++count;
      const int j = current - 1;
      const bool own = lane == (j & 63);
#pragma unroll
      for (int r = 0; r < NR; ++r)
        if (r == (j >> 6)) {
          rpar[r] = own ? parent : rpar[r];
          rtok[r] = own ? token : rtok[r];
          rdep[r] = own ? depth : rdep[r];
        }
    }
    // ---- sibling (rank + 1) takes over the popped slot, or the slot dies; the winner lane rescans its slots
    uint32_t shi = NONE, slo = NONE;
    double slw = 0.0;
    if (rank + 1 < kk) {
      slw = (logw - (double)lp_r) + (double)lp_r1;
      shi = key_bits(-((float)slw + pr));
      slo = pack_fields(mode, parent, depth, rank + 1);
    } else {
      --alive;
    }
    const bool me = lane == win;
    if (row < RR) {
#pragma unroll
      for (int rr = 0; rr < RR; ++rr)
        if (rr == row) {
          khi[rr] = me ? shi : khi[rr];
          klo[rr] = me ? slo : klo[rr];
          klw[rr] = me ? slw : klw[rr];
        }
    } else if (me) {
      const int slot = row * WAVE + win;
      fhi[slot] = shi;
      flo[slot] = slo;
      flogw[slot] = slw;
    }
    {
      uint32_t bh = khi[0], bl = klo[0];
      int br = 0;
      double bw = klw[0];
#pragma unroll
      for (int rr = 1; rr < RR; ++rr) {
        const bool lt = khi[rr] < bh || (khi[rr] == bh && klo[rr] < bl);
        bh = lt ? khi[rr] : bh;
        bl = lt ? klo[rr] : bl;
        br = lt ? rr : br;
        bw = lt ? klw[rr] : bw;
      }
      if (tail > RR * WAVE && me) {  // rows in LDS
        for (int s = RR * WAVE + lane; s < tail; s += WAVE) {
          const uint32_t h = fhi[s], l = flo[s];
          if (h < bh || (h == bh && l < bl)) {
            bh = h;
            bl = l;
            br = s / WAVE;
            bw = flogw[s];
          }
        }
      }
      lhi = me ? bh : lhi;
      llo = me ? bl : llo;
      lrow = me ? br : lrow;
      lbw = me ? bw : lbw;
    }
    // ---- child (depth + 1, rank 0) of the node just reached, in the next slot
    if (depth < L) {
      if (tail < cap) {
        const double clw = logw + (double)lp_c;
        const uint32_t chi = key_bits(-((float)clw + pr));
        const uint32_t clo = pack_fields(mode, current, depth + 1, 0);
        const int tr = tail / WAVE;
        const bool mine = lane == (tail & 63);
        if (tr < RR) {
#pragma unroll
          for (int rr = 0; rr < RR; ++rr)
            if (rr == tr) {
              khi[rr] = mine ? chi : khi[rr];
              klo[rr] = mine ? clo : klo[rr];
              klw[rr] = mine ? clw : klw[rr];
            }
        } else if (mine) {
          fhi[tail] = chi;
          flo[tail] = clo;
          flogw[tail] = clw;
        }
        const bool better = mine && (chi < lhi || (chi == lhi && clo < llo));
        lhi = better ? chi : lhi;
        llo = better ? clo : llo;
        lrow = better ? tr : lrow;
        lbw = better ? clw : lbw;
        ++tail;
        ++alive;
      } else {
        overflow = true;
        break;
      }
    }
    prefetch();
  }
  if (overflow && lane == 0 && a.err) atomicOr(a.err, 1);
  // node table to LDS for the outputs
  if (lane == 0) {
    npar[0] = -1;
    ntok[0] = 0;
    ndep[0] = 0;
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int j = 64 * r + lane;
    if (j < count) {
      npar[j + 1] = rpar[r];
      ntok[j + 1] = rtok[r];
      ndep[j + 1] = rdep[r];
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();

  write_tree(a, b, lane, count, npar, ntok, ndep);
}

// ---- single-mode DDTree heap (inference/hf/tree_build_ext.py:31-46 SingleEntry / SingleGreater, :118-156
// build_single; inference/sglang/patches/sglang-v0.5.22-mfd.patch:1295-1328 build_single_one): key -logw in
// fp64, ties by the rank tuple (the ranks along the prefix, compared as Python tuples: element by element,
// a proper prefix first); every pop is a new node. A key is the order-preserving bits of the fp64 key in two
// 32-bit halves; the rank tuples are compared only for entries whose keys are equal, by climbing the node
// table from both entries to their first common parent.

__device__ __forceinline__ uint64_t dkey_bits(double key) {
  const uint64_t b = __builtin_bit_cast(uint64_t, key + 0.0);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
// fields of a single-mode entry: parent 12b | depth 6b | rank 10b (as pack_fields with mode 0)
// Rank tuple of an entry (parent p, depth d, rank r): the ranks of p's root path (nodes at depths 1..d-1)
// followed by r. True when entry fa's tuple orders before fb's.
__device__ bool ranks_less(uint32_t fa, uint32_t fb, const int32_t* npar, const int32_t* nrank) {
  int ap = (int)((fa >> 16) & 0xFFF), ad = (int)((fa >> 10) & 0x3F), ar = (int)(fa & 0x3FF);
  int bp = (int)((fb >> 16) & 0xFFF), bd = (int)((fb >> 10) & 0x3F), br = (int)(fb & 0x3FF);
  const int m = min(ad, bd);
  // the position (parent, rank) of each tuple's prefix of length m
  for (int d = ad; d > m; --d) {
    ar = nrank[ap];
    ap = max(npar[ap], 0);
  }
  for (int d = bd; d > m; --d) {
    br = nrank[bp];
    bp = max(npar[bp], 0);
  }
  if (ap == bp && ar == br) return ad < bd;  // one tuple is a prefix of the other
  // both prefixes have length m: climb to the first common parent, where the ranks differ
  for (int it = 0; it < 64 && ap != bp; ++it) {
    ar = nrank[ap];
    ap = max(npar[ap], 0);
    br = nrank[bp];
    bp = max(npar[bp], 0);
  }
  return ar < br;
}

// LDS layout (dynamic): frontier logw f64 [cap], key halves u32 [cap] x 2, fields u32 [cap], lp f32 [L k],
// ids i32 [L k], node parent / token / depth / rank i32 [budget + 1].
__global__ __launch_bounds__(WAVE) void build_single_kernel(BuildArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char smem[];
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int L = a.L, kk = a.k, cap = a.cap, budget = a.budget;
  const int nlp = L * kk;
  double* flogw = reinterpret_cast<double*>(smem);
  uint32_t* fhi = reinterpret_cast<uint32_t*>(flogw + cap);
  uint32_t* flo = fhi + cap;
  uint32_t* ffd = flo + cap;
  float* slp = reinterpret_cast<float*>(ffd + cap);
  int32_t* sid = reinterpret_cast<int32_t*>(slp + nlp);
  int32_t* npar = sid + nlp;
  int32_t* ntok = npar + (budget + 1);
  int32_t* ndep = ntok + (budget + 1);
  int32_t* nrank = ndep + (budget + 1);

  const float* lpb = a.lp + (int64_t)b * nlp;
  if (a.ids_int64) {
    stage_lds(reinterpret_cast<const int32_t*>(lpb), reinterpret_cast<int32_t*>(slp), nlp, lane);
    stage_lds(static_cast<const int64_t*>(a.ids) + (int64_t)b * nlp, sid, nlp, lane);
  } else {
    stage_lds(reinterpret_cast<const int32_t*>(lpb), reinterpret_cast<int32_t*>(slp), nlp, lane);
    stage_lds(static_cast<const int32_t*>(a.ids) + (int64_t)b * nlp, sid, nlp, lane);
  }
  uint32_t lhi = NONE, llo = NONE, lfd = NONE;  // this lane's best live slot
  int lslot = lane;
  if (lane == 0) {
    const double lw = (double)lpb[0];
    const uint64_t kb = dkey_bits(-lw);
    lhi = (uint32_t)(kb >> 32);
    llo = (uint32_t)kb;
    lfd = pack_fields(0, 0, 1, 0);
    fhi[0] = lhi;
    flo[0] = llo;
    ffd[0] = lfd;
    flogw[0] = lw;
    npar[0] = -1;
    ntok[0] = 0;
    ndep[0] = 0;
    nrank[0] = 0;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();

  // entry x orders before entry y
  auto before = [&](uint32_t xh, uint32_t xl, uint32_t xf, uint32_t yh, uint32_t yl, uint32_t yf) {
    if (xh != yh) return xh < yh;
    if (xl != yl) return xl < yl;
    return ranks_less(xf, yf, npar, nrank);
  };
  int count = 0, tail = 1, alive = 1;
  bool overflow = false;
  for (int iter = 0; iter < cap && alive > 0 && count < budget; ++iter) {
    // ---- pop: smallest key; equal keys by rank tuple
    const uint32_t mh = wave_min_u32(lhi);
    uint64_t tie = __builtin_amdgcn_ballot_w64(lhi == mh);
    if (__builtin_popcountll(tie) > 1) {
      const uint32_t ml = wave_min_u32(lhi == mh ? llo : NONE);
      tie = __builtin_amdgcn_ballot_w64(lhi == mh && llo == ml);
    }
    int win = (int)__builtin_ctzll(tie);
    for (uint64_t rest = tie & (tie - 1); rest; rest &= rest - 1) {
      const int j = (int)__builtin_ctzll(rest);
      if (ranks_less(__builtin_amdgcn_readlane(lfd, j), __builtin_amdgcn_readlane(lfd, win), npar, nrank)) win = j;
    }
    const uint32_t f = __builtin_amdgcn_readlane(lfd, win);
    const int slot = __builtin_amdgcn_readlane(lslot, win);
    const int parent = (int)((f >> 16) & 0xFFF);
    const int depth = (int)((f >> 10) & 0x3F);
    const int rank = (int)(f & 0x3FF);
    const int base = (depth - 1) * kk;
    const double logw = flogw[slot];
    const int token = sid[base + rank];
    const float lp_r = slp[base + rank];
    const float lp_r1 = slp[base + min(rank + 1, kk - 1)];
    const float lp_c = slp[min(depth, L - 1) * kk];
    // ---- the popped prefix is a new node
    const int current = ++count;
    if (lane == 0) {
      npar[current] = parent;
      ntok[current] = token;
      ndep[current] = depth;
      nrank[current] = rank;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    // ---- sibling (rank + 1) takes over the popped slot, or the slot dies; its lane rescans its slots
    uint32_t shi = NONE, slo = NONE, sfd = NONE;
    double slw = 0.0;
    if (rank + 1 < kk) {
      slw = (logw - (double)lp_r) + (double)lp_r1;
      const uint64_t kb = dkey_bits(-slw);
      shi = (uint32_t)(kb >> 32);
      slo = (uint32_t)kb;
      sfd = pack_fields(0, parent, depth, rank + 1);
    } else {
      --alive;
    }
    if (lane == (slot & 63)) {
      fhi[slot] = shi;
      flo[slot] = slo;
      ffd[slot] = sfd;
      flogw[slot] = slw;
      uint32_t bh = NONE, bl = NONE, bf = NONE;
      int bsl = lane;
      for (int s = lane; s < tail; s += WAVE) {
        const uint32_t h = fhi[s], l = flo[s], fd = ffd[s];
        if (h != NONE && (bh == NONE || before(h, l, fd, bh, bl, bf))) {
          bh = h;
          bl = l;
          bf = fd;
          bsl = s;
        }
      }
      lhi = bh;
      llo = bl;
      lfd = bf;
      lslot = bsl;
    }
    // ---- child (depth + 1, rank 0) of the new node, in the next slot
    if (depth < L) {
      if (tail < cap) {
        const double clw = logw + (double)lp_c;
        const uint64_t kb = dkey_bits(-clw);
        const uint32_t chi = (uint32_t)(kb >> 32), clo = (uint32_t)kb;
        const uint32_t cfd = pack_fields(0, current, depth + 1, 0);
        if (lane == (tail & 63)) {
          fhi[tail] = chi;
          flo[tail] = clo;
          ffd[tail] = cfd;
          flogw[tail] = clw;
          if (lhi == NONE || before(chi, clo, cfd, lhi, llo, lfd)) {
            lhi = chi;
            llo = clo;
            lfd = cfd;
            lslot = tail;
          }
        }
        ++tail;
        ++alive;
      } else {
        overflow = true;
        break;
      }
    }
  }
  if (overflow && lane == 0 && a.err) atomicOr(a.err, 1);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  write_tree(a, b, lane, count, npar, ntok, ndep);
}

}  // namespace

extern "C" int mfd_build_mixture_smem_bytes(int K, int L, int k, int budget, int* cap_out) {
  // frontier bound: each pop pushes at most one new slot (the child; the sibling reuses the popped slot)
  const int64_t cap = (int64_t)K + 2LL * K * budget + 2;
  const int64_t c = cap > 4096 ? 4096 : cap;
  if (cap_out) *cap_out = (int)c;
  return (int)(c * 16 + (int64_t)K * L * k * 8 + 64 + (int64_t)(budget + 1) * 12);
}

namespace {
template <int NR>
int launch_build(const BuildArgs& a, int smem, hipStream_t st) {
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&build_mixture_kernel<NR>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return mfd_set_hip_error(e);
    attr_set = true;
  }
  hipLaunchKernelGGL(build_mixture_kernel<NR>, dim3(a.bs), dim3(WAVE), smem, st, a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
}  // namespace

extern "C" int mfd_build_mixture(const float* top_logp, const void* top_ids, int ids_int64, const float* log_prior,
                                 int bs, int K, int L, int k, int budget, int64_t* tree_out, int64_t* counts_out,
                                 int8_t* anc8_out, int32_t* err_flag, void* stream) {
  if (bs < 0 || K < 1 || K > 16 || L < 1 || L > 63 || k < 1 || k > 1023 || budget < 0 || budget > 4095)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_build_mixture: K=%d (1..16) L=%d (1..63) k=%d (1..1023) budget=%d "
                         "(0..4095)", K, L, k, budget);
  if (bs == 0) return MFD_OK;
  if (!top_logp || !top_ids || !tree_out || !counts_out)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_build_mixture: null pointer");
  int cap = 0;
  const int smem = mfd_build_mixture_smem_bytes(K, L, k, budget, &cap);
  if (smem > 160 * 1024)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_build_mixture: %d bytes of LDS needed (K L k too large)", smem);
  BuildArgs a{top_logp, top_ids, ids_int64, log_prior, bs, K, L, k, budget, cap, tree_out, counts_out, anc8_out,
              err_flag};
  hipStream_t st = static_cast<hipStream_t>(stream);
  // register slots of the node table per lane: 64 NR >= budget
  if (budget <= 64) return launch_build<1>(a, smem, st);
  if (budget <= 128) return launch_build<2>(a, smem, st);
  if (budget <= 256) return launch_build<4>(a, smem, st);
  if (budget <= 512) return launch_build<8>(a, smem, st);
  if (budget <= 1024) return launch_build<16>(a, smem, st);
  if (budget <= 2048) return launch_build<32>(a, smem, st);
  return launch_build<64>(a, smem, st);
}

extern "C" int mfd_build_single_smem_bytes(int L, int k, int budget, int* cap_out) {
  // every pop adds at most the child slot; the sibling reuses the popped slot
  const int64_t cap = (int64_t)budget + 2;
  if (cap_out) *cap_out = (int)cap;
  return (int)(cap * 20 + (int64_t)L * k * 8 + (int64_t)(budget + 1) * 16);
}

extern "C" int mfd_build_single(const float* top_logp, const void* top_ids, int ids_int64, int bs, int L, int k,
                                int budget, int64_t* tree_out, int64_t* counts_out, int8_t* anc8_out,
                                int32_t* err_flag, void* stream) {
  if (bs < 0 || L < 1 || L > 63 || k < 1 || k > 1023 || budget < 0 || budget > 4095)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_build_single: L=%d (1..63) k=%d (1..1023) budget=%d (0..4095)", L, k,
                         budget);
  if (bs == 0) return MFD_OK;
  if (!top_logp || !top_ids || !tree_out || !counts_out)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_build_single: null pointer");
  int cap = 0;
  const int smem = mfd_build_single_smem_bytes(L, k, budget, &cap);
  if (smem > 160 * 1024)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_build_single: %d bytes of LDS needed (L k or budget too large)", smem);
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&build_single_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return mfd_set_hip_error(e);
    attr_set = true;
  }
  BuildArgs a{top_logp, top_ids, ids_int64, nullptr, bs, 1, L, k, budget, cap, tree_out, counts_out, anc8_out, err_flag};
  hipLaunchKernelGGL(build_single_kernel, dim3(bs), dim3(WAVE), smem, static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
