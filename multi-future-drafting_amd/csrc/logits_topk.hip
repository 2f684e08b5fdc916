// Logits step of tree construction for gfx950: per row of bf16 draft logits, the top-k (value descending,
// token id ascending) and their log-probabilities value - log Z.
//
// Reference semantics: inference/hf/tree_logits.py:34-46 (torch.topk on the bf16 logits, log Z from an
// fp32 online max/sum) and the fp32 variant inference/hf/ddtree.py:240-245. Here log Z is computed with a
// reduction whose result does not depend on the order in which the hardware combines partial sums:
//   the row is cut into chunks of MFD_LZ_CHUNK elements; chunk c has max m_c and
//   S_c = sum_x lz_term(max(x - m_c, -80)) ~ rint(e^d 2^30)   (exact integers, summed exactly)
//   Z  = sum_c S_c * exp_det(m_c - m) in chunk order (fp64),  log Z = float(m + log_det(Z * 2^-30)).
// lz_term (a 256-entry table of 2^(i/256) 2^30, lz_table.h, and a 2-term polynomial), exp_det and log_det
// use only IEEE +, *, fma, division and exact power-of-two scaling, with contraction disabled, so the CPU
// restatement produces the same bits (and log Z agrees with an fp64 logsumexp to about one fp32 ulp).
//
// Kernel 1: one workgroup per (row, chunk): 8192 elements in registers (32 per thread), chunk max, the
//           fixed-point sum, and the chunk's top-k. k <= 32: threshold selection (ballot radix select over
//           the lane maxima, then only the keys above the threshold are compacted and ranked); larger k:
//           per-thread sorted lists, merged per wave, then per block.
// Kernel 2: one wave per row: merges the chunks' candidates (for k <= 32 staged in LDS first), combines the
//           sums, writes log-probs / ids.
#include "mfd_common.h"
#include "lz_table.h"

#define MFD_LZ_CHUNK 8192

namespace {

constexpr int CHUNK = MFD_LZ_CHUNK;
constexpr int NT = 256;
constexpr int PER = CHUNK / NT;  // 32 elements per thread
constexpr int FINAL_STAGE = 2048;  // candidates per row staged in LDS by the k <= 32 merge (16 KB)
constexpr int KMAX = 256;  // a thread holds 32 elements: its 32-entry list keeps all of them for k > 32

__device__ __forceinline__ float pow2i(int k) { return __uint_as_float((uint32_t)(k + 127) << 23); }

__device__ float exp_det(float d) {
#pragma clang fp contract(off)
  const float k = __builtin_rintf(d * 1.44269504088896341f);
  float r = __builtin_fmaf(k, -0.693145751953125f, d);
  r = __builtin_fmaf(k, -1.42860676533018592e-06f, r);
  float p = 2.48015873015873016e-05f;
  p = __builtin_fmaf(p, r, 1.98412698412698413e-04f);
  p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return p * pow2i((int)k);
}

__device__ double log_det(double z) {
#pragma clang fp contract(off)
  int e;
  double f = frexp(z, &e);
  if (f < 0.70710678118654752440) {
    f = f * 2.0;
    e -= 1;
  }
  const double s = (f - 1.0) / (f + 1.0);
  const double s2 = s * s;
  double p = 1.0 / 23.0;
  p = __builtin_fma(p, s2, 1.0 / 21.0);
  p = __builtin_fma(p, s2, 1.0 / 19.0);
  p = __builtin_fma(p, s2, 1.0 / 17.0);
  p = __builtin_fma(p, s2, 1.0 / 15.0);
  p = __builtin_fma(p, s2, 1.0 / 13.0);
  p = __builtin_fma(p, s2, 1.0 / 11.0);
  p = __builtin_fma(p, s2, 1.0 / 9.0);
  p = __builtin_fma(p, s2, 1.0 / 7.0);
  p = __builtin_fma(p, s2, 1.0 / 5.0);
  p = __builtin_fma(p, s2, 1.0 / 3.0);
  p = __builtin_fma(p, s2, 1.0);
  const double logf_ = 2.0 * s * p;
  const double de = (double)e;
  return __builtin_fma(de, 6.93147180369123816490e-01, __builtin_fma(de, 1.90821492927058770002e-10, logf_));
}

// fixed-point contribution of one element (an exact integer <= 2^30)
// Per-element term of the fixed-point sum, rint(e^d 2^30) for d = max(x - m, -80) to within float rounding:
// j = rint(d 256/ln2), r = d - j ln2/256 (ln2/256 in two parts; the first has 9 bits, so j times it is
// exact), e^r ~ 1 + r + r^2/2 (|r| <= ln2/512: truncation 4e-10, below float rounding), times tab[j mod 256]
// = 2^((j mod 256)/256) 2^30 (lz_table.h), scaled by 2^floor(j/256). 15 VALU and one LDS read per element
// (the 9-term polynomial of exp_det took 22 VALU); the CPU oracle computes the same sequence.
__device__ __forceinline__ float lz_term(float x, float m, const float* tab) {
#pragma clang fp contract(off)
  float d = x - m;
  d = d > -80.0f ? d : -80.0f;
  const float jf = __builtin_rintf(d * 369.329925537109375f);
  const int j = (int)jf;
  float r = __builtin_fmaf(jf, -0x1.63p-9f, d);
  r = __builtin_fmaf(jf, 0x1.bd0106p-21f, r);
  const float p = __builtin_fmaf(__builtin_fmaf(r, 0.5f, 1.0f), r, 1.0f);
  const float e = tab[j & 255] * p;
  return __builtin_rintf(__builtin_ldexpf(e, j >> 8));
}
__device__ const float lz_table_g[256] = {MFD_LZ_TABLE_INIT};

// candidate key: larger = better (value descending, then token id ascending)
__device__ __forceinline__ uint64_t cand_key(float x, uint32_t idx) {
  return ((uint64_t)float_order_key(x + 0.0f) << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const int lane = threadIdx.x & 63;
  const int src = (lane ^ mask) << 2;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const uint64_t o = shfl_xor_u64(v, m);
    v = o > v ? o : v;
  }
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(((threadIdx.x & 63) ^ m) << 2,
                                                                          __builtin_bit_cast(int, v))));
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const uint64_t b = shfl_xor_u64(__builtin_bit_cast(uint64_t, v), m);
    v += __builtin_bit_cast(double, b);
  }
  return v;
}

// one list per thread, merged across the wave: k rounds of "best head wins"
template <int KT>
__device__ void wave_topk(const uint64_t (&list)[KT], int k, uint64_t* out /* LDS, k entries */) {
  int head = 0;
  for (int i = 0; i < k; ++i) {
    uint64_t mine = 0;
#pragma unroll
    for (int j = 0; j < KT; ++j)
      if (j == head) mine = list[j];
    const uint64_t best = wave_max_u64(mine);
    if (best != 0 && mine == best) ++head;  // keys are unique (they contain the token id)
    if ((threadIdx.x & 63) == 0) out[i] = best;
  }
}

struct ChunkArgs {
  const uint16_t* logits;
  int64_t row_stride;
  int rows, V, k, nchunks;
  float* ws_m;        // [rows * nchunks]
  double* ws_s;       // [rows * nchunks]
  uint64_t* ws_cand;  // [rows * nchunks * k]
};

template <int KT>
__global__ __launch_bounds__(NT) void topk_logz_chunk_kernel(ChunkArgs a) {
  __shared__ uint64_t wcand[NT / 64][KMAX];
  __shared__ float wmax[NT / 64];
  __shared__ double wsum[NT / 64];
  const int tid = threadIdx.x;
  __shared__ float lz_tab[256];  // per-element term table (read after the first barrier below)
  static_assert(NT == 256, "one table entry per thread");
  lz_tab[tid] = lz_table_g[tid];
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int row = blockIdx.x / a.nchunks;
  const int chunk = blockIdx.x % a.nchunks;
  const int64_t c0 = (int64_t)chunk * CHUNK;
  const uint16_t* src = a.logits + (int64_t)row * a.row_stride;

  // element (j, e) of this thread: index c0 + 2048 j + 8 tid + e (increasing with (j, e))
  u16x8 raw[PER / 8];
#pragma unroll
  for (int j = 0; j < PER / 8; ++j) {
    const int64_t i0 = c0 + 2048 * j + 8 * tid;
    if (i0 + 8 <= a.V) {
      raw[j] = *reinterpret_cast<const u16x8*>(src + i0);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) raw[j][e] = (i0 + e < a.V) ? src[i0 + e] : (uint16_t)0xFF80u;  // -inf
    }
  }
  float mx = -INFINITY;
  uint64_t list[KT];
#pragma unroll
  for (int i = 0; i < KT; ++i) list[i] = 0;
#pragma unroll
  for (int j = 0; j < PER / 8; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = bf2f(raw[j][e]);
      mx = fmaxf(mx, x);
      const int64_t idx = c0 + 2048 * j + 8 * tid + e;
      if (idx < a.V) {
        uint64_t key = cand_key(x, (uint32_t)idx);
        if (key > list[KT - 1]) {
          // insertion into the descending list (unrolled compare-and-shift)
#pragma unroll
          for (int s = 0; s < KT; ++s) {
            const uint64_t cur = list[s];
            const bool take = key > cur;
            list[s] = take ? key : cur;
            key = take ? cur : key;
          }
        }
      }
    }
  // chunk max
  mx = wave_max_f(mx);
  if (lane == 0) wmax[w] = mx;
  __syncthreads();
  float m = wmax[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) m = fmaxf(m, wmax[i]);
  // fixed-point sum against the chunk max (exact integers: any summation order gives the same value)
  double acc = 0.0;
  if (m != -INFINITY) {
#pragma unroll
    for (int j = 0; j < PER / 8; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (double)lz_term(bf2f(raw[j][e]), m, lz_tab);
  }
  acc = wave_sum_d(acc);
  // per-wave top-k, then the first wave merges the 4 wave lists
  wave_topk<KT>(list, a.k, wcand[w]);
  if (lane == 0) wsum[w] = acc;
  __syncthreads();
  const int64_t slot = (int64_t)row * a.nchunks + chunk;
  if (w == 0) {
    // the 4 waves' k candidates, spread over the lanes as sorted per-lane lists (at most 4 k / 64 <= 16 per
    // lane), then k rounds of argmax
    uint64_t l2[KT];
#pragma unroll
    for (int i = 0; i < KT; ++i) l2[i] = 0;
    for (int t = lane; t < (NT / 64) * a.k; t += 64) {
      uint64_t key = wcand[t % (NT / 64)][t / (NT / 64)];
#pragma unroll
      for (int s = 0; s < KT; ++s) {
        const uint64_t cur = l2[s];
        const bool take = key > cur;
        l2[s] = take ? key : cur;
        key = take ? cur : key;
      }
    }
    uint64_t* out = a.ws_cand + slot * a.k;
    int head = 0;
    for (int i = 0; i < a.k; ++i) {
      uint64_t mine = 0;
#pragma unroll
      for (int j = 0; j < KT; ++j)
        if (j == head) mine = l2[j];
      const uint64_t best = wave_max_u64(mine);
      if (best != 0 && mine == best) ++head;
      if (lane == 0) out[i] = best;
    }
    if (lane == 0) {
      double tot = 0.0;
#pragma unroll
      for (int i = 0; i < NT / 64; ++i) tot += wsum[i];
      a.ws_m[slot] = m;
      a.ws_s[slot] = tot;
    }
  }
}

// ---- fast path for k <= 32 ----------------------------------------------------------------------------
// Chunk keys are 32-bit: the upper half is the order key of the bf16 value (the upper 16 bits of
// float_order_key of the widened value; its lower 16 bits are 0 for positive and 0xFFFF for negative values,
// so nothing is lost), the lower half is 0xFFFF minus the element's index within the chunk. Larger key =
// larger value, then smaller token id; keys are unique within a chunk and never 0 (0 marks an empty lane).
__device__ __forceinline__ uint32_t chunk_key(uint16_t raw, int local_idx) {
  // float_order_key of the widened value as (bits ^ (sign ? ~0 : 0x80000000)), then the index half
  const uint32_t b = __float_as_uint(bf2f(raw) + 0.0f);
  const uint32_t flip = (uint32_t)((int32_t)b >> 31) | 0x80000000u;
  return ((b ^ flip) & 0xFFFF0000u) | (uint32_t)(0xFFFF - local_idx);
}
// the 64-bit candidate key (cand_key) of a chunk key
__device__ __forceinline__ uint64_t global_key(uint32_t ck, int64_t c0) {
  const uint32_t hi = (ck & 0xFFFF0000u) | ((ck & 0x80000000u) ? 0u : 0xFFFFu);
  const int64_t idx = c0 + (0xFFFF - (int)(ck & 0xFFFFu));
  return ((uint64_t)hi << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}
// The k-th largest of the 64 lane values (0 = no value): the largest t with #{lanes: v >= t} >= k, found
// bit by bit from the top with ballots; 0 when fewer than k lanes hold a value. Wave-uniform.
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t v, int k) {
  uint32_t t = 0;
#pragma unroll
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t c = t | (1u << bit);
    if (__builtin_popcountll(__builtin_amdgcn_ballot_w64(v >= c)) >= k) t = c;
  }
  return t;
}
// the same for 64-bit values: the high words first; the low words only decide among the lanes tied at the
// boundary, and only when more of them are tied than are still needed
__device__ __forceinline__ uint64_t wave_kth_largest64(uint64_t v, int k) {
  const uint32_t hi = (uint32_t)(v >> 32);
  const uint32_t th = wave_kth_largest(hi, k);
  const int above = __builtin_popcountll(__builtin_amdgcn_ballot_w64(hi > th));
  const int tied = __builtin_popcountll(__builtin_amdgcn_ballot_w64(hi == th));
  const int need = k - above;
  uint32_t tl = 0;
  if (tied > need) tl = wave_kth_largest(hi == th ? (uint32_t)v : 0u, need);
  return ((uint64_t)th << 32) | tl;
}
template <int N>
__device__ __forceinline__ uint32_t row_ror32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + N, 0xF, 0xF, false);
}
// wave maximum of a float (uniform result): DPP rotations within rows of 16, then the four row maxima
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, __uint_as_float(row_ror32<1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(row_ror32<2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(row_ror32<4>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(row_ror32<8>(__float_as_uint(v))));
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
// wave sum of a 64-bit integer (uniform result)
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    switch (m) {
      case 1: lo = row_ror32<1>(lo); hi = row_ror32<1>(hi); break;
      case 2: lo = row_ror32<2>(lo); hi = row_ror32<2>(hi); break;
      case 4: lo = row_ror32<4>(lo); hi = row_ror32<4>(hi); break;
      default: lo = row_ror32<8>(lo); hi = row_ror32<8>(hi); break;
    }
    v += ((uint64_t)hi << 32) | lo;
  }
  uint64_t s = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    s += ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((uint32_t)(v >> 32), 16 * r) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((uint32_t)v, 16 * r);
  return s;
}

// Kernel 1 (k <= 32): one workgroup per (row, chunk), 32 elements per thread. Each wave finds the k-th
// largest of its 64 lane maxima (t_w); the chunk's top k are all >= t* = max_w t_w (the wave attaining
// t* alone has k elements >= t*), and at most 32 k elements per wave pass that test (only the <= k lanes
// whose maximum is >= t_w hold any). The passing keys are compacted per wave into LDS, then one wave keeps a
// running top k over them in 64-lane passes. The fixed-point sum is the same integer sum as in
// topk_logz_chunk_kernel (exact, so its value does not depend on the summation order).
template <int KS>
__global__ __launch_bounds__(NT) void topk_small_chunk_kernel(ChunkArgs a) {
  constexpr int WCAP = 32 * KS;
  __shared__ uint32_t wcand[NT / 64][WCAP];
  __shared__ uint32_t wthr[NT / 64];
  __shared__ uint32_t wn[NT / 64];
  __shared__ float wmax[NT / 64];
  __shared__ uint64_t wsum[NT / 64];
  __shared__ uint32_t keep_buf[64];
  const int tid = threadIdx.x;
  __shared__ float lz_tab[256];  // per-element term table (read after the first barrier below)
  static_assert(NT == 256, "one table entry per thread");
  lz_tab[tid] = lz_table_g[tid];
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int row = blockIdx.x / a.nchunks;
  const int chunk = blockIdx.x % a.nchunks;
  const int64_t c0 = (int64_t)chunk * CHUNK;
  const uint16_t* src = a.logits + (int64_t)row * a.row_stride;
  const int k = a.k;

  // element (j, e) of this thread: chunk index 2048 j + 8 tid + e; past the row end it reads as -inf and
  // gets key 0
  u16x8 raw[PER / 8];
#pragma unroll
  for (int j = 0; j < PER / 8; ++j) {
    const int64_t i0 = c0 + 2048 * j + 8 * tid;
    if (i0 + 8 <= a.V) {
      raw[j] = *reinterpret_cast<const u16x8*>(src + i0);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) raw[j][e] = (i0 + e < a.V) ? src[i0 + e] : (uint16_t)0xFF80u;
    }
  }
  const int nvalid = (int)min((int64_t)CHUNK, (int64_t)a.V - c0);
  float mx = -INFINITY;
  uint32_t key[PER];
#pragma unroll
  for (int j = 0; j < PER / 8; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      mx = fmaxf(mx, bf2f(raw[j][e]));
      key[8 * j + e] = chunk_key(raw[j][e], 2048 * j + 8 * tid + e);
    }
  if (nvalid < CHUNK) {  // the row's last chunk: elements past the row end get key 0
#pragma unroll
    for (int j = 0; j < PER / 8; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (2048 * j + 8 * tid + e >= nvalid) key[8 * j + e] = 0u;
  }
  uint32_t lmax = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) lmax = key[i] > lmax ? key[i] : lmax;
  const uint32_t tw = wave_kth_largest(lmax, k);
  mx = wave_max_dpp(mx);
  if (lane == 0) {
    wthr[w] = tw;
    wmax[w] = mx;
  }
  __syncthreads();
  uint32_t tstar = wthr[0];
  float m = wmax[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) {
    tstar = wthr[i] > tstar ? wthr[i] : tstar;
    m = fmaxf(m, wmax[i]);
  }
  // compaction of the keys >= t* of this wave (ballot + lane rank)
  uint32_t nc = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const bool take = key[i] != 0u && key[i] >= tstar;
    const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
    if (mk) {
      if (take) wcand[w][nc + __builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0))] = key[i];
      nc += (uint32_t)__builtin_popcountll(mk);
    }
  }
  // fixed-point sum: two terms (each <= 2^30) add exactly in 32 bits, pairs accumulate in 64 bits
  uint64_t acc = 0;
  if (m != -INFINITY) {
#pragma unroll
    for (int j = 0; j < PER / 8; ++j)
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        acc += (uint64_t)((uint32_t)lz_term(bf2f(raw[j][e]), m, lz_tab) + (uint32_t)lz_term(bf2f(raw[j][e + 1]), m, lz_tab));
  }
  acc = wave_sum_u64(acc);
  if (lane == 0) {
    wn[w] = nc;
    wsum[w] = acc;
  }
  __syncthreads();
  if (w != 0) return;
  const int n0 = (int)wn[0], n1 = (int)wn[1], n2 = (int)wn[2], n3 = (int)wn[3];
  const int total = n0 + n1 + n2 + n3;
  auto fetch = [&](int i) -> uint32_t {
    if (i >= total) return 0u;
    if (i < n0) return wcand[0][i];
    i -= n0;
    if (i < n1) return wcand[1][i];
    i -= n1;
    if (i < n2) return wcand[2][i];
    return wcand[3][i - n2];
  };
  // running top k: lanes hold the kept keys (low lanes) and the next unseen candidates
  uint32_t v = fetch(lane);
  int next = 64;
  uint64_t km;
  for (;;) {
    const uint32_t t = wave_kth_largest(v, k);
    const bool keep = v != 0u && v >= t;
    km = __builtin_amdgcn_ballot_w64(keep);
    if (next >= total) break;
    const int nk = __builtin_popcountll(km);
    if (keep) keep_buf[__builtin_amdgcn_mbcnt_hi((uint32_t)(km >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)km, 0))] = v;
    __builtin_amdgcn_wave_barrier();
    v = lane < nk ? keep_buf[lane] : fetch(next + lane - nk);
    __builtin_amdgcn_wave_barrier();
    next += 64 - nk;
  }
  const int64_t slot = (int64_t)row * a.nchunks + chunk;
  uint64_t* out = a.ws_cand + slot * k;
  const bool keep = (km >> lane) & 1ull;
  const int pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(km >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)km, 0));
  if (keep) out[pos] = global_key(v, c0);
  const int nk = __builtin_popcountll(km);
  if (lane >= nk && lane < k) out[lane] = 0;
  if (lane == 0) {
    a.ws_m[slot] = m;
    a.ws_s[slot] = (double)(wsum[0] + wsum[1] + wsum[2] + wsum[3]);
  }
}

// Kernel 2 (k <= 32): one wave per row. The chunk terms S_c exp_det(m_c - m) are formed in parallel and
// summed in chunk order by one lane (the same operations as topk_logz_final_kernel); the row's top k are
// kept over the chunk candidates in 64-lane passes (64-bit keys), then ranked for the output order.
struct FinalArgs {
  int rows, k, nchunks;
  const float* ws_m;
  const double* ws_s;
  const uint64_t* ws_cand;
  float* out_logp;     // [rows, k]
  void* out_ids;       // [rows, k] int32 or int64
  int ids_int64;
  float* out_logz;     // [rows] or null
  const int32_t* vocab_ids;  // [V] token id of each logit column, or null (column = token id)
};

constexpr int FINAL_CAND = 8192;  // candidates of one row staged in LDS (nchunks * k)

__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t hi = (uint32_t)(key >> 32);
  return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
}

// one wave per row
__global__ __launch_bounds__(64) void topk_logz_final_kernel(FinalArgs a) {
#pragma clang fp contract(off)
  __shared__ uint64_t cand[FINAL_CAND];
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const int n = a.nchunks * a.k;
  const uint64_t* src = a.ws_cand + (int64_t)row * n;
  for (int t = lane; t < n; t += 64) cand[t] = src[t];
  // log Z in chunk order (lane 0)
  float logz = -INFINITY;
  if (lane == 0) {
    const float* mc = a.ws_m + (int64_t)row * a.nchunks;
    const double* sc = a.ws_s + (int64_t)row * a.nchunks;
    float m = -INFINITY;
    for (int c = 0; c < a.nchunks; ++c) m = fmaxf(m, mc[c]);
    if (m != -INFINITY) {
      double z = 0.0;
      for (int c = 0; c < a.nchunks; ++c) {
        if (mc[c] == -INFINITY) continue;
        float d = mc[c] - m;
        d = d > -80.0f ? d : -80.0f;
        const double f = (double)exp_det(d);
        const double t = sc[c] * f;
        z = z + t;
      }
      logz = (float)((double)m + log_det(z * 9.31322574615478515625e-10));
    }
  }
  logz = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, logz)));
  // k rounds of wave argmax; keys are unique (they contain the token id), the winner is removed
  for (int i = 0; i < a.k; ++i) {
    uint64_t mine = 0;
    int where = -1;
    for (int t = lane; t < n; t += 64) {
      const uint64_t c = cand[t];
      if (c > mine) {
        mine = c;
        where = t;
      }
    }
    const uint64_t best = wave_max_u64(mine);
    if (best != 0 && mine == best) cand[where] = 0;
    if (lane == 0) {
      const float x = best ? key_value(best) : -INFINITY;
      uint32_t idx = best ? 0xFFFFFFFFu - (uint32_t)best : 0u;
      if (best && a.vocab_ids) idx = (uint32_t)a.vocab_ids[idx];
      a.out_logp[(int64_t)row * a.k + i] = x - logz;
      if (a.ids_int64)
        static_cast<int64_t*>(a.out_ids)[(int64_t)row * a.k + i] = (int64_t)idx;
      else
        static_cast<int32_t*>(a.out_ids)[(int64_t)row * a.k + i] = (int32_t)idx;
    }
  }
  if (lane == 0 && a.out_logz) a.out_logz[row] = logz;
}


__global__ __launch_bounds__(64) void topk_small_final_kernel(FinalArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char fsm[];
  double* terms = reinterpret_cast<double*>(fsm);  // [nchunks]
  uint64_t* keep_buf = reinterpret_cast<uint64_t*>(terms + a.nchunks);  // [64]
  uint64_t* cand = keep_buf + 64;  // [nchunks k] when nchunks k <= FINAL_STAGE: the row's candidates
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const int nch = a.nchunks;
  const int k = a.k;
  const float* mc = a.ws_m + (int64_t)row * nch;
  const double* sc = a.ws_s + (int64_t)row * nch;
  const int n = nch * k;
  const uint64_t* src = a.ws_cand + (int64_t)row * n;
  // the candidates are loaded first (up to 4 per lane into registers, in flight while log Z is formed) and
  // staged in LDS, so that the selection passes below read no global memory
  const bool staged = n <= FINAL_STAGE;
  uint64_t pre[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) pre[x] = (staged && x * 64 + lane < n) ? src[x * 64 + lane] : 0ull;
  // chunk c's term S_c exp_det(m_c - m) is formed by lane c % 64; lane 0 adds them in chunk order (a chunk
  // whose maximum is -inf adds +0, which leaves the non-negative sum unchanged)
  float m = -INFINITY;
  for (int c = lane; c < nch; c += 64) m = fmaxf(m, mc[c]);
  m = wave_max_dpp(m);
  float logz = -INFINITY;
  if (m != -INFINITY) {
    auto term = [&](int c) -> double {
      const float mcc = mc[c];
      if (mcc == -INFINITY) return 0.0;
      float d = mcc - m;
      d = d > -80.0f ? d : -80.0f;
      const double f = (double)exp_det(d);
      return sc[c] * f;
    };
    double z = 0.0;
    if (nch <= 64) {
      const double t = lane < nch ? term(lane) : 0.0;
      const uint64_t tb = __builtin_bit_cast(uint64_t, t);
      for (int c = 0; c < nch; ++c) {
        const uint64_t xb = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((uint32_t)(tb >> 32), c) << 32) |
                            (uint32_t)__builtin_amdgcn_readlane((uint32_t)tb, c);
        z = z + __builtin_bit_cast(double, xb);
      }
    } else {
      for (int c = lane; c < nch; c += 64) terms[c] = term(c);
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
      for (int c = 0; c < nch; ++c) z = z + terms[c];
    }
    logz = (float)((double)m + log_det(z * 9.31322574615478515625e-10));
  }
  if (k == 0) {
    if (lane == 0 && a.out_logz) a.out_logz[row] = logz;
    return;
  }
  if (staged) {
#pragma unroll
    for (int x = 0; x < 4; ++x)
      if (x * 64 + lane < n) cand[x * 64 + lane] = pre[x];
    for (int i = 256 + lane; i < n; i += 64) cand[i] = src[i];
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
  }
  const uint64_t* cs = staged ? cand : src;
  uint64_t v = lane < n ? cs[lane] : 0ull;
  int next = 64;
  uint64_t km;
  for (;;) {
    const uint64_t t = wave_kth_largest64(v, k);
    const bool keep = v != 0ull && v >= t;
    km = __builtin_amdgcn_ballot_w64(keep);
    if (next >= n) break;
    const int nk = __builtin_popcountll(km);
    if (keep) keep_buf[__builtin_amdgcn_mbcnt_hi((uint32_t)(km >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)km, 0))] = v;
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    const int i = next + lane - nk;
    v = lane < nk ? keep_buf[lane] : (i < n ? cs[i] : 0ull);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    next += 64 - nk;
  }
  // output position of a kept key = number of kept keys larger than it
  const bool keep = (km >> lane) & 1ull;
  const int nk = __builtin_popcountll(km);
  int rank = 0;
  uint64_t rest = km;
  while (rest) {
    const int j = (int)__builtin_ctzll(rest);
    rest &= rest - 1;
    const uint64_t vj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((uint32_t)(v >> 32), j) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane((uint32_t)v, j);
    rank += vj > v ? 1 : 0;
  }
  auto put = [&](int pos, uint64_t key) {
    const float x = key ? key_value(key) : -INFINITY;
    uint32_t idx = key ? 0xFFFFFFFFu - (uint32_t)key : 0u;
    if (key && a.vocab_ids) idx = (uint32_t)a.vocab_ids[idx];
    a.out_logp[(int64_t)row * k + pos] = x - logz;
    if (a.ids_int64)
      static_cast<int64_t*>(a.out_ids)[(int64_t)row * k + pos] = (int64_t)idx;
    else
      static_cast<int32_t*>(a.out_ids)[(int64_t)row * k + pos] = (int32_t)idx;
  };
  if (keep) put(rank, v);
  if (lane >= nk && lane < k) put(lane, 0ull);
  if (lane == 0 && a.out_logz) a.out_logz[row] = logz;
}

}  // namespace

extern "C" int64_t mfd_topk_logz_workspace_bytes(int rows, int V, int k) {
  const int64_t nchunks = ((int64_t)V + CHUNK - 1) / CHUNK;
  return (int64_t)rows * nchunks * (4 + 8 + 8 * (int64_t)(k > 0 ? k : 1)) + 64;
}

static int topk_logz_impl(const uint16_t* logits, int rows, int V, int64_t row_stride, int k, float* out_logp,
                          void* out_ids, int ids_int64, float* out_logz, const int32_t* vocab_ids, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  if (rows < 0 || V < 1 || k < 0 || k > V)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_topk_logz: bad sizes rows=%d V=%d k=%d", rows, V, k);
  if (k > KMAX) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_topk_logz: k=%d > %d", k, KMAX);
  if ((int64_t)((V + CHUNK - 1) / CHUNK) * (k > 0 ? k : 1) > FINAL_CAND)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_topk_logz: V=%d with k=%d exceeds the merge capacity", V, k);
  if (row_stride < V || (row_stride % 8) != 0 || (reinterpret_cast<uintptr_t>(logits) % 16) != 0)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_topk_logz: rows must be 16-byte aligned (stride %lld)",
                         (long long)row_stride);
  if (rows == 0) return MFD_OK;
  if (!logits || (k > 0 && (!out_logp || !out_ids)) || (k == 0 && !out_logz))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_topk_logz: null pointer");
  const int64_t need = mfd_topk_logz_workspace_bytes(rows, V, k);
  if (!workspace || workspace_bytes < need)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_topk_logz: workspace of %lld bytes needed", (long long)need);
  const int nchunks = (V + CHUNK - 1) / CHUNK;
  const int kk = k > 0 ? k : 1;
  char* ws = static_cast<char*>(workspace);
  uint64_t* cand = reinterpret_cast<uint64_t*>(ws);
  double* s = reinterpret_cast<double*>(ws + (int64_t)rows * nchunks * kk * 8);
  float* m = reinterpret_cast<float*>(ws + (int64_t)rows * nchunks * (kk * 8 + 8));
  ChunkArgs ca{logits, row_stride, rows, V, kk, nchunks, m, s, cand};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((int64_t)rows * nchunks));
  if (kk <= 32) {
    if (kk <= 8)
      hipLaunchKernelGGL(topk_small_chunk_kernel<8>, grid, dim3(NT), 0, st, ca);
    else if (kk <= 16)
      hipLaunchKernelGGL(topk_small_chunk_kernel<16>, grid, dim3(NT), 0, st, ca);
    else
      hipLaunchKernelGGL(topk_small_chunk_kernel<32>, grid, dim3(NT), 0, st, ca);
    MFD_CHECK_LAUNCH();
    static bool attr_set = false;
    if (!attr_set) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_small_final_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      if (e != hipSuccess) return mfd_set_hip_error(e);
      attr_set = true;
    }
    FinalArgs fa{rows, k, nchunks, m, s, cand, out_logp, out_ids, ids_int64, out_logz, vocab_ids};
    const int ncand = nchunks * k;
    const size_t smem = (size_t)(nchunks + 64 + (ncand <= FINAL_STAGE ? ncand : 0)) * sizeof(double);
    hipLaunchKernelGGL(topk_small_final_kernel, dim3(rows), dim3(64), smem, st, fa);
    MFD_CHECK_LAUNCH();
    return MFD_OK;
  }
  if (kk <= 8)
    hipLaunchKernelGGL(topk_logz_chunk_kernel<8>, grid, dim3(NT), 0, st, ca);
  else if (kk <= 16)
    hipLaunchKernelGGL(topk_logz_chunk_kernel<16>, grid, dim3(NT), 0, st, ca);
  else
    hipLaunchKernelGGL(topk_logz_chunk_kernel<32>, grid, dim3(NT), 0, st, ca);
  MFD_CHECK_LAUNCH();
  // k == 0 (log Z only): one candidate per chunk is still kept by kernel 1; kernel 2 takes none of them
  FinalArgs fa{rows, k, nchunks, m, s, cand, out_logp, out_ids, ids_int64, out_logz, vocab_ids};
  hipLaunchKernelGGL(topk_logz_final_kernel, dim3(rows), dim3(64), 0, st, fa);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

extern "C" int mfd_topk_logz(const uint16_t* logits, int rows, int V, int64_t row_stride, int k, float* out_logp,
                             void* out_ids, int ids_int64, float* out_logz, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  return topk_logz_impl(logits, rows, V, row_stride, k, out_logp, out_ids, ids_int64, out_logz, nullptr, workspace,
                        workspace_bytes, stream);
}

extern "C" int mfd_topk_logz_vocab(const uint16_t* logits, int rows, int V, int64_t row_stride, int k,
                                   float* out_logp, void* out_ids, int ids_int64, float* out_logz,
                                   const int32_t* vocab_ids, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!vocab_ids) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_topk_logz_vocab: vocab_ids is required");
  return topk_logz_impl(logits, rows, V, row_stride, k, out_logp, out_ids, ids_int64, out_logz, vocab_ids, workspace,
                        workspace_bytes, stream);
}
