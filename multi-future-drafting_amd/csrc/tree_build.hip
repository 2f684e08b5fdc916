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
// The frontier, the (parent, token) -> node table and the pop records live in registers (one wave);
// batches of pops that provably come next in the heap's order are taken in one step (see the kernel).
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
  int hsize;             // (parent, token) hash slots of the batch step, a power of two (0: no batch steps)
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
constexpr int BMAX = 64;  // entries one batch pops at most (one per lane)
constexpr int BMIN = 6;   // frontier heads below sigma from which a batch is tried

constexpr uint64_t HEMPTY = ~0ull;
__device__ __forceinline__ uint32_t hash_pt(int parent, int token) {
  uint32_t x = (uint32_t)token * 0x9E3779B1u + (uint32_t)parent * 0x85EBCA77u;
  x ^= x >> 15;
  x *= 0x2C1B3C6Du;
  x ^= x >> 12;
  return x;
}
// (key, fields) pair order
__device__ __forceinline__ bool pair_lt(uint32_t ka, uint32_t fa, uint32_t kb, uint32_t fb) {
  return ka < kb || (ka == kb && fa < fb);
}

// A frontier slot holds the head of a sibling list: the next rank not yet popped of the children of one
// popped entry (or of the root, per mode), with its logw, key and the key of its own rank-0 child (NONE at
// depth L). The heap pops the smallest (key, fields) head; its sibling replaces it and its child list opens
// in a new slot. This is the reference heap's frontier: an entry there is pushed when its elder sibling or
// its parent entry is popped.
//
// Batches. Keys never decrease from an entry to the entries it generates (a child adds lp <= 0 to logw; a
// sibling adds lp_{r+1} - lp_r <= 0, up to an fp64 rounding that is checked), so the pop order is the
// (key bits, fields) order of all entries. With sigma = the smallest child key over the frontier, every
// frontier entry with key < sigma, together with the frontier minimum f1, pops before anything a pop can
// generate; the siblings of a head below sigma are such entries too. When at least BMIN heads are below
// sigma, one step pops that whole prefix: the candidates (heads, and their siblings while below sigma; at
// most 64) are ordered by (key, fields), all their parents being known nodes, so the order is the heap's,
// ties included; the batch is cut after an entry whose next sibling would order before the next batch entry
// (an fp64 rounding that put that sibling's key below its elder's: the walk stops before such a sibling) and
// after the pop that creates node number budget. Otherwise the step pops f1 alone.
//
// LDS layout (dynamic): slot logw f64 [cap], slot key u32 [cap], slot fields u32 [cap], slot child key
// u32 [cap], slot last-popped rank i32 [cap] (rows >= RR always; register rows are copied in for a batch),
// candidate logw f64 [64], key / fields / slot u32 [64], records (token, lp bits) [K L k], prior f32 [16],
// node parent / token / depth i32 [budget + 1], counter i32 [4].
// NR = register slots per lane of the node table (64 NR >= budget).
//
// A sequential pop needs no LDS round trip: every lane keeps its best slot's key, fields, row and logw in
// registers, and after each pop every lane prefetches the records its best entry will need if popped.
template <int NR>
__global__ __launch_bounds__(WAVE) void build_mixture_kernel(BuildArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char smem[];
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int K = a.K, L = a.L, kk = a.k, cap = a.cap, budget = a.budget;
  const int nlp = K * L * kk;
  const int HS = a.hsize;
  double* flogw = reinterpret_cast<double*>(smem);
  double* clw = flogw + cap;
  uint64_t* hkey = reinterpret_cast<uint64_t*>(clw + BMAX);
  uint32_t* fhi = reinterpret_cast<uint32_t*>(hkey + HS);
  uint32_t* flo = fhi + cap;
  uint32_t* fck = flo + cap;
  int32_t* fmax = reinterpret_cast<int32_t*>(fck + cap);
  int32_t* hid = fmax + cap;
  int32_t* hmin = hid + HS;
  uint32_t* ck = reinterpret_cast<uint32_t*>(hmin + HS);
  uint32_t* cf = ck + BMAX;
  int32_t* cs = reinterpret_cast<int32_t*>(cf + BMAX);
  int2* rec = reinterpret_cast<int2*>(cs + BMAX);
  float* sprior = reinterpret_cast<float*>(rec + nlp);
  int32_t* npar = reinterpret_cast<int32_t*>(sprior + 16);
  int32_t* ntok = npar + (budget + 1);
  int32_t* ndep = ntok + (budget + 1);
  int32_t* scnt = ndep + (budget + 1);

  const float* lpb = a.lp + (int64_t)b * nlp;
  if (a.ids_int64)
    stage_records(lpb, static_cast<const int64_t*>(a.ids) + (int64_t)b * nlp, rec, nlp, lane);
  else
    stage_records(lpb, static_cast<const int32_t*>(a.ids) + (int64_t)b * nlp, rec, nlp, lane);
  for (int s = lane; s < cap; s += WAVE) fmax[s] = -1;
  for (int h = lane; h < HS; h += WAVE) {
    hkey[h] = HEMPTY;
    hid[h] = -1;
    hmin[h] = 0x7FFFFFFF;
  }
  auto lp_at = [&](int m, int row, int r) __attribute__((always_inline)) {
    return __int_as_float(rec[(m * L + row) * kk + r].y);
  };

  // register frontier rows; unused slots hold NONE keys and never win
  uint32_t khi[RR], klo[RR], kck[RR];
  double klw[RR];
#pragma unroll
  for (int rr = 0; rr < RR; ++rr) {
    khi[rr] = NONE;
    klo[rr] = NONE;
    kck[rr] = NONE;
    klw[rr] = 0.0;
  }
  // this lane's best live slot (key bits, fields, row, logw) and the smallest child key of its slots
  uint32_t lhi = NONE, llo = NONE, lcm = NONE;
  int lrow = 0;
  double lbw = 0.0;
  if (lane < K) sprior[lane] = a.prior ? a.prior[(int64_t)b * K + lane] : 0.f;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // seed: one entry per mode (rank 0 at depth 1 under the root) in slot m, which lane m owns (K <= 16)
  if (lane < K) {
    const float pr = sprior[lane];
    const double lw = (double)lp_at(lane, 0, 0);
    lhi = key_bits(-((float)lw + pr));
    llo = pack_fields(lane, 0, 1, 0);
    khi[0] = lhi;
    klo[0] = llo;
    klw[0] = lw;
    kck[0] = L > 1 ? key_bits(-((float)(lw + (double)lp_at(lane, 1, 0)) + pr)) : NONE;
    lbw = lw;
    lcm = kck[0];
  }
  int32_t rpar[NR], rtok[NR], rdep[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    rpar[r] = -1;  // never equals a parent id
    rtok[r] = 0;
    rdep[r] = 0;
  }

  // records of this lane's best entry (mode m, depth d, rank r): token and lp of (m, d, r), lp of rank r + 1,
  // lp of (m, d + 1, 0) and of (m, d + 2, 0), prior of m. Lanes without a live slot read entry 0.
  int ptok;
  float plp, plp1, plpc, plpn, ppr;
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
    plpn = __int_as_float(rec[(m * L + min(dm1 + 2, L - 1)) * kk].y);
    ppr = sprior[m];
  };
  // best slot and smallest child key of this lane over all its rows
  auto rescan = [&](int tail) __attribute__((always_inline)) {
    uint32_t bh = khi[0], bl = klo[0], bc = kck[0];
    int br = 0;
    double bw = klw[0];
#pragma unroll
    for (int rr = 1; rr < RR; ++rr) {
      const bool lt = pair_lt(khi[rr], klo[rr], bh, bl);
      bh = lt ? khi[rr] : bh;
      bl = lt ? klo[rr] : bl;
      br = lt ? rr : br;
      bw = lt ? klw[rr] : bw;
      bc = umin32(bc, kck[rr]);
    }
    for (int s = RR * WAVE + lane; s < tail; s += WAVE) {  // rows in LDS
      const uint32_t h = fhi[s], l = flo[s];
      bc = umin32(bc, fck[s]);
      if (pair_lt(h, l, bh, bl)) {
        bh = h;
        bl = l;
        br = s / WAVE;
        bw = flogw[s];
      }
    }
    lhi = bh;
    llo = bl;
    lrow = br;
    lbw = bw;
    lcm = bc;
  };
  prefetch();

  int count = 0, tail = K, alive = K, hashed = 0, next_check = 0, gap = 2;
  bool overflow = false;
  // Batch step: pops the prefix of the frontier order below sigma at once (see above). Returns false, with
  // nothing changed, when the candidates exceed 64 or a list has more than WALK of them.
  auto batch_step = [&](uint32_t f1, uint32_t mh, uint32_t sigma) -> bool {
    constexpr int WALK = 8;
    if (tail > RR * WAVE) return false;
    // register rows to LDS; the nodes made by sequential pops since the last batch into the hash table
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) {
      const int s = rr * WAVE + lane;
      if (s < tail) {
        fhi[s] = khi[rr];
        flo[s] = klo[rr];
        fck[s] = kck[rr];
        flogw[s] = klw[rr];
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int id = 64 * r + lane + 1;
      if (id > hashed && id <= count) {
        const uint64_t key64 = ((uint64_t)(uint32_t)rpar[r] << 32) | (uint32_t)rtok[r];
        int slot = (int)(hash_pt(rpar[r], rtok[r]) & (uint32_t)(HS - 1));
        for (int probe = 0; probe < HS; ++probe) {
          const uint64_t old = atomicCAS(reinterpret_cast<unsigned long long*>(&hkey[slot]),
                                         (unsigned long long)HEMPTY, (unsigned long long)key64);
          if (old == HEMPTY || old == key64) break;
          slot = (slot + 1) & (HS - 1);
        }
        hid[slot] = id;
      }
    }
    hashed = count;
    // candidates: heads below sigma (f1 in any case) and their siblings while below sigma and not below
    // their elder, at most WALK per list; walked in registers (a frontier with LDS rows is not batched)
    uint32_t hk[RR][WALK];
    double wv[RR][WALK];
    int nc[RR];
    bool too_long = false;
    {
      float lpv[RR][WALK + 1];
      float prr[RR];
#pragma unroll
      for (int rr = 0; rr < RR; ++rr) {
        const bool q = khi[rr] != NONE && (khi[rr] < sigma || (khi[rr] == mh && klo[rr] == f1));
        nc[rr] = q ? 1 : 0;
        const uint32_t fl0 = q ? klo[rr] : 0u;
        const int m = (int)(fl0 >> 28), row = q ? (int)((fl0 >> 10) & 0x3F) - 1 : 0;
        const int r0 = (int)(fl0 & 0x3FF);
#pragma unroll
        for (int t = 0; t <= WALK; ++t) lpv[rr][t] = lp_at(m, row, min(r0 + t, kk - 1));
        prr[rr] = sprior[m];
      }
#pragma unroll
      for (int rr = 0; rr < RR; ++rr) {
        const int r0 = (int)(klo[rr] & 0x3FF);
        hk[rr][0] = khi[rr];
        wv[rr][0] = klw[rr];
#pragma unroll
        for (int t = 1; t <= WALK; ++t) {
          if (nc[rr] == t && r0 + t < kk) {
            const double wn = (wv[rr][t - 1] - (double)lpv[rr][t - 1]) + (double)lpv[rr][t];
            const uint32_t hn = key_bits(-((float)wn + prr[rr]));
            if (hn < sigma && hn >= hk[rr][t - 1]) {
              if (t < WALK) {
                hk[rr][t] = hn;
                wv[rr][t] = wn;
                nc[rr] = t + 1;
              } else {
                too_long = true;
              }
            }
          }
        }
      }
    }
    // positions: exclusive prefix of the per-lane counts over the lanes (bit by bit through ballots)
    int c_lane = 0;
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) c_lane += nc[rr];
    const uint64_t below_l = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    int base = 0, nb = 0;
#pragma unroll
    for (int bit = 0; bit < 5; ++bit) {
      const uint64_t bb = __builtin_amdgcn_ballot_w64((c_lane >> bit) & 1);
      base += __builtin_popcountll(bb & below_l) << bit;
      nb += __builtin_popcountll(bb) << bit;
    }
    if (nb > BMAX || __builtin_amdgcn_ballot_w64(too_long) != 0) return false;
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) {
      const int s = rr * WAVE + lane;
#pragma unroll
      for (int t = 0; t < WALK; ++t)
        if (t < nc[rr]) {
          ck[base + t] = hk[rr][t];
          cf[base + t] = (klo[rr] & ~0x3FFu) | (uint32_t)((klo[rr] & 0x3FF) + t);
          clw[base + t] = wv[rr][t];
          cs[base + t] = s;
        }
      base += nc[rr];
    }
    __syncthreads();
    uint32_t ekey = NONE, efld = NONE;
    double ew = 0.0;
    int eslot = 0;
    if (lane < nb) {
      ekey = ck[lane];
      efld = cf[lane];
      ew = clw[lane];
      eslot = cs[lane];
    }
    // order: lane i takes the candidate of rank i. Every lane compares its candidate with all of them, read
    // four at a time (the same LDS words for every lane: broadcast reads); the tail up to a multiple of four
    // holds (NONE, NONE), which orders after every candidate.
    const int nb4 = (nb + 3) & ~3;
    if (lane >= nb && lane < nb4) {
      ck[lane] = NONE;
      cf[lane] = NONE;
    }
    __syncthreads();
    // (key, fields) as one 64-bit word; equal words (only with repeated ids in a top list) rank by lane
    const uint64_t me64 = ((uint64_t)ekey << 32) | efld;
    int rank_o = 0;
    for (int j = 0; j < nb4; j += 4) {
      const uint4 k4 = *reinterpret_cast<const uint4*>(ck + j);
      const uint4 f4 = *reinterpret_cast<const uint4*>(cf + j);
      const uint64_t c0 = ((uint64_t)k4.x << 32) | f4.x, c1 = ((uint64_t)k4.y << 32) | f4.y;
      const uint64_t c2 = ((uint64_t)k4.z << 32) | f4.z, c3 = ((uint64_t)k4.w << 32) | f4.w;
      rank_o += (int)(c0 < me64) + (int)(c1 < me64) + (int)(c2 < me64) + (int)(c3 < me64);
      rank_o += (int)(c0 == me64 && j < lane) + (int)(c1 == me64 && j + 1 < lane) + (int)(c2 == me64 && j + 2 < lane) +
                (int)(c3 == me64 && j + 3 < lane);
    }
    __syncthreads();
    if (lane < nb) {
      ck[rank_o] = ekey;
      cf[rank_o] = efld;
      clw[rank_o] = ew;
      cs[rank_o] = eslot;
    }
    __syncthreads();
    const bool cand = lane < nb;
    if (cand) {
      ekey = ck[lane];
      efld = cf[lane];
      ew = clw[lane];
      eslot = cs[lane];
    }
    const int m = cand ? (int)(efld >> 28) : 0;
    const int parent = (int)((efld >> 16) & 0xFFF);
    const int depth = cand ? (int)((efld >> 10) & 0x3F) : 1;
    const int rank = cand ? (int)(efld & 0x3FF) : 0;
    const float pr = sprior[m];
    const int token = cand ? rec[(m * L + depth - 1) * kk + rank].x : 0;
    const bool has_next = cand && rank + 1 < kk;
    double nw = 0.0;
    uint32_t nkey = NONE, nfld = NONE;
    if (has_next) {
      nw = (ew - (double)lp_at(m, depth - 1, rank)) + (double)lp_at(m, depth - 1, rank + 1);
      nkey = key_bits(-((float)nw + pr));
      nfld = (efld & ~0x3FFu) | (uint32_t)(rank + 1);
    }
    // cut after an entry whose list's next sibling orders before the next batch entry
    if (cand) atomicMax(&fmax[eslot], rank);
    __syncthreads();
    const bool last_of_list = cand && fmax[eslot] == rank;
    const uint32_t kn = lane + 1 < nb ? ck[lane + 1] : NONE;
    const uint32_t fn = lane + 1 < nb ? cf[lane + 1] : NONE;
    __syncthreads();
    if (last_of_list) fmax[eslot] = -1;
    const uint64_t cuts =
        __builtin_amdgcn_ballot_w64(last_of_list && lane + 1 < nb && has_next && pair_lt(nkey, nfld, kn, fn));
    if (cuts != 0) nb = (int)__builtin_ctzll(cuts) + 1;
    // nodes: (parent, token) in the hash table; the first lane of a new prefix creates it, ids in batch order,
    // and the batch ends with the pop that creates node number budget
    const bool contend = lane < nb;
    int slot = 0;
    bool existing = false, lost = false;
    if (contend) {
      const uint64_t key64 = ((uint64_t)(uint32_t)parent << 32) | (uint32_t)token;
      slot = (int)(hash_pt(parent, token) & (uint32_t)(HS - 1));
      bool found = false;
      for (int probe = 0; probe < HS; ++probe) {
        const uint64_t old = atomicCAS(reinterpret_cast<unsigned long long*>(&hkey[slot]),
                                       (unsigned long long)HEMPTY, (unsigned long long)key64);
        if (old == HEMPTY || old == key64) {
          found = true;
          break;
        }
        slot = (slot + 1) & (HS - 1);
      }
      lost = !found;
      existing = hid[slot] >= 0;
      if (!existing) atomicMin(&hmin[slot], lane);
    }
    if (__builtin_amdgcn_ballot_w64(lost) != 0) overflow = true;  // kept wave-uniform
    __syncthreads();
    const bool creator = contend && !existing && hmin[slot] == lane;
    const uint64_t cre = __builtin_amdgcn_ballot_w64(creator);
    const int need = budget - count;
    if (__builtin_popcountll(cre) >= need) {
      uint64_t c = cre;
      for (int i = 1; i < need; ++i) c &= c - 1;
      nb = min(nb, (int)__builtin_ctzll(c) + 1);
    }
    const bool live = lane < nb;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int id = count + 1 + __builtin_popcountll(cre & below);
    if (live && creator) {
      hid[slot] = id;
      npar[id] = parent;
      ntok[id] = token;
      ndep[id] = depth;
    }
    // a creator cut off above releases the slot for later steps (the key stays, without a node)
    if (creator && !live) hmin[slot] = 0x7FFFFFFF;
    __syncthreads();
    const int enode = live ? (creator ? id : hid[slot]) : 0;
    const int count_new = count + __builtin_popcountll(cre & (nb >= 64 ? ~0ull : ((1ull << nb) - 1)));
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int nid = 64 * r + lane + 1;
      if (nid > count && nid <= count_new) {
        rpar[r] = npar[nid];
        rtok[r] = ntok[nid];
        rdep[r] = ndep[nid];
      }
    }
    count = count_new;
    hashed = count;
    // each list moves its head past its last popped entry; popped entries below depth L open their children's
    // lists in new slots
    if (live) atomicMax(&fmax[eslot], rank);
    __syncthreads();
    const bool last = live && fmax[eslot] == rank;
    __syncthreads();
    if (last) {
      fmax[eslot] = -1;
      if (has_next) {
        fhi[eslot] = nkey;
        flo[eslot] = nfld;
        flogw[eslot] = nw;
        fck[eslot] = depth < L ? key_bits(-((float)(nw + (double)lp_at(m, depth, 0)) + pr)) : NONE;
      } else {
        fhi[eslot] = NONE;
        flo[eslot] = NONE;
        fck[eslot] = NONE;
      }
    }
    alive -= __builtin_popcountll(__builtin_amdgcn_ballot_w64(last && !has_next));
    const bool opens = live && depth < L;
    const uint64_t op = __builtin_amdgcn_ballot_w64(opens);
    const int nnew = __builtin_popcountll(op);
    if (tail + nnew > cap) {
      overflow = true;
      return true;
    }
    if (opens) {
      const int s = tail + __builtin_popcountll(op & below);
      const double w0 = ew + (double)lp_at(m, depth, 0);
      fhi[s] = key_bits(-((float)w0 + pr));
      flo[s] = pack_fields(m, enode, depth + 1, 0);
      flogw[s] = w0;
      fck[s] = depth + 1 < L ? key_bits(-((float)(w0 + (double)lp_at(m, depth + 1, 0)) + pr)) : NONE;
    }
    tail += nnew;
    alive += nnew;
    __syncthreads();
    // LDS rows back to the registers, then every lane's best and prefetch
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) {
      const int s = rr * WAVE + lane;
      const bool in = s < tail;
      khi[rr] = in ? fhi[s] : NONE;
      klo[rr] = in ? flo[s] : NONE;
      kck[rr] = in ? fck[s] : NONE;
      klw[rr] = in ? flogw[s] : 0.0;
    }
    rescan(tail);
    prefetch();
    __syncthreads();
    return true;
  };
  // every iteration pops at least one frontier entry and at most cap entries are ever pushed: bounded loop
  for (int iter = 0; iter < cap && alive > 0 && count < budget; ++iter) {
    // ---- the frontier minimum f1: the lane holding the smallest (key bits, fields)
    const uint32_t mh = wave_min_u32(lhi);
    const uint64_t tie = __builtin_amdgcn_ballot_w64(lhi == mh);
    int win = (int)__builtin_ctzll(tie);
    if (__builtin_popcountll(tie) > 1) {
      const uint32_t ml = wave_min_u32(lhi == mh ? llo : NONE);
      win = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(lhi == mh && llo == ml));
    }
    const uint32_t f = __builtin_amdgcn_readlane(llo, win);
    // ---- batch step when enough heads lie below sigma. Checked 4 steps after a batch, then at gaps that
    //      double (up to 32) while the checks find none.
    bool batched = false;
    if (iter == next_check && HS > 0) {
      const uint32_t sigma = wave_min_u32(lcm);
      int nheads = 0;
#pragma unroll
      for (int rr = 0; rr < RR; ++rr)
        nheads += __builtin_popcountll(__builtin_amdgcn_ballot_w64(khi[rr] < sigma));
      if (nheads >= BMIN) batched = batch_step(f, mh, sigma);
      if (overflow) break;
      gap = batched ? 4 : min(2 * gap, 32);
      next_check = iter + gap;
    }
    if (batched) continue;
    // ---- sequential pop of f1
    const int row = __builtin_amdgcn_readlane(lrow, win);
    const double logw = readlane_f64(lbw, win);
    const int token = __builtin_amdgcn_readlane(ptok, win);
    const float lp_r = readlane_f32(plp, win);
    const float lp_r1 = readlane_f32(plp1, win);
    const float lp_c = readlane_f32(plpc, win);
    const float lp_n = readlane_f32(plpn, win);
    const float pr = readlane_f32(ppr, win);
    const int mode = (int)(f >> 28);
    const int parent = (int)((f >> 16) & 0xFFF);
    const int depth = (int)((f >> 10) & 0x3F);
    const int rank = (int)(f & 0x3FF);
    // node of (parent, token), or a new node
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
    // sibling (rank + 1) takes over the popped slot, or the slot dies; the winner lane rescans its slots
    uint32_t shi = NONE, slo = NONE, sck = NONE;
    double slw = 0.0;
    if (rank + 1 < kk) {
      slw = (logw - (double)lp_r) + (double)lp_r1;
      shi = key_bits(-((float)slw + pr));
      slo = pack_fields(mode, parent, depth, rank + 1);
      sck = depth < L ? key_bits(-((float)(slw + (double)lp_c) + pr)) : NONE;
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
          kck[rr] = me ? sck : kck[rr];
          klw[rr] = me ? slw : klw[rr];
        }
    } else if (me) {
      const int slot = row * WAVE + win;
      fhi[slot] = shi;
      flo[slot] = slo;
      fck[slot] = sck;
      flogw[slot] = slw;
    }
    if (me) rescan(tail);
    // child (depth + 1, rank 0) of the node just reached, in the next slot
    if (depth < L) {
      if (tail < cap) {
        const double clw0 = logw + (double)lp_c;
        const uint32_t chi = key_bits(-((float)clw0 + pr));
        const uint32_t clo = pack_fields(mode, current, depth + 1, 0);
        const uint32_t cck = depth + 1 < L ? key_bits(-((float)(clw0 + (double)lp_n) + pr)) : NONE;
        const int tr = tail / WAVE;
        const bool mine = lane == (tail & 63);
        if (tr < RR) {
#pragma unroll
          for (int rr = 0; rr < RR; ++rr)
            if (rr == tr) {
              khi[rr] = mine ? chi : khi[rr];
              klo[rr] = mine ? clo : klo[rr];
              kck[rr] = mine ? cck : kck[rr];
              klw[rr] = mine ? clw0 : klw[rr];
            }
        } else if (mine) {
          fhi[tail] = chi;
          flo[tail] = clo;
          fck[tail] = cck;
          flogw[tail] = clw0;
        }
        const bool better = mine && pair_lt(chi, clo, lhi, llo);
        lhi = better ? chi : lhi;
        llo = better ? clo : llo;
        lrow = better ? tr : lrow;
        lbw = better ? clw0 : lbw;
        lcm = mine ? umin32(lcm, cck) : lcm;
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
  __syncthreads();
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

// (parent, token) hash slots of the batch step: the power of two >= 2 (budget + 1) + 128
static int hash_slots(int budget) {
  int hs = 1;
  while (hs < 2 * (budget + 1) + 128) hs <<= 1;
  return hs;
}

// LDS of the mixture kernel with hs hash slots (0: no batch steps)
static int64_t mixture_smem(int K, int L, int k, int budget, int64_t cap, int hs) {
  return cap * 24 + (int64_t)hs * 16 + (int64_t)BMAX * 20 + (int64_t)K * L * k * 8 + 64 + (int64_t)(budget + 1) * 12 +
         16;
}
// hash slots the kernel gets: the batch steps' table when it fits in LDS beside the rest, else none
static int mixture_hash_slots(int K, int L, int k, int budget, int64_t cap) {
  return mixture_smem(K, L, k, budget, cap, hash_slots(budget)) <= 160 * 1024 ? hash_slots(budget) : 0;
}

extern "C" int mfd_build_mixture_smem_bytes(int K, int L, int k, int budget, int* cap_out) {
  // frontier bound: each pop pushes at most one new slot (the child; the sibling reuses the popped slot)
  const int64_t cap = (int64_t)K + 2LL * K * budget + 2;
  const int64_t c = ((cap > 4096 ? 4096 : cap) + 1) & ~1LL;  // even: keeps the candidate arrays 16-byte aligned
  if (cap_out) *cap_out = (int)c;
  return (int)mixture_smem(K, L, k, budget, c, mixture_hash_slots(K, L, k, budget, c));
}

namespace {
template <int NR>
int launch_build(const BuildArgs& a, int smem, hipStream_t st) {
  const int rc = mfd_set_max_lds(reinterpret_cast<const void*>(&build_mixture_kernel<NR>), 160 * 1024);
  if (rc != MFD_OK) return rc;
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
              err_flag, mixture_hash_slots(K, L, k, budget, cap)};
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
  {
    const int rc = mfd_set_max_lds(reinterpret_cast<const void*>(&build_single_kernel), 160 * 1024);
    if (rc != MFD_OK) return rc;
  }
  BuildArgs a{top_logp, top_ids, ids_int64, nullptr, bs, 1, L, k, budget, cap, tree_out, counts_out, anc8_out, err_flag};
  hipLaunchKernelGGL(build_single_kernel, dim3(bs), dim3(WAVE), smem, static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
