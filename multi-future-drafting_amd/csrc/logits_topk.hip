// Logits step of tree construction for gfx950: per row of bf16 draft logits, the top-k (value descending,
// token id ascending) and their log-probabilities value - log Z.
//
// Reference semantics: inference/hf/tree_logits.py:34-46 (torch.topk on the bf16 logits, log Z from an
// fp32 online max/sum) and the fp32 variant inference/hf/ddtree.py:240-245. Here log Z is computed in one
// fixed order of IEEE operations, so that the CPU restatement produces the same bits:
//   the row is cut into pieces of MFD_LZ_PIECE = 2048 elements; piece c has max m_c, and its element
//   512 j + 8 l + e belongs to lane l (l < 64, j < 4, e < 8), which sums its 32 elements in (j, e) order
//   starting from 0:
//     s = fma(E(x), C, s),  C = E(-m_c)             if -60 <= m_c < 64 (E: e^x for every bf16 x with
//                                                    2^-25 <= |x| < 128, rounded to float: exp_bf16_table.h)
//     s = s + exp_det(max(x - m_c, -80))            otherwise (an all -inf piece sums to 0)
//   the 64 lane sums are added pairwise over lane distances 32, 16, 8, 4, 2, 1 (every lane ends with the
//   same value S_c);
//   Z = sum_c S_c exp_det(max(m_c - m, -80)) in piece order (fp64), log Z = float(m + log_det(Z)).
// exp_det and log_det use only IEEE +, *, fma, division and exact power-of-two scaling, with contraction
// disabled; log Z agrees with an fp64 logsumexp to about one fp32 ulp.
// The table index of a bf16 bit pattern b is min(max(rotl16(b, 1) - 0x6600, 0), 8191), formed for two
// elements at once with packed 16-bit operations; the table sits in LDS (32 KB, staged once per workgroup
// with direct-to-LDS loads).
//
// Kernel 1 (k <= 32): one wave per piece, no workgroup barrier after the table: the piece's maximum, its sum
//           S_c and its top k (the k-th largest 16-bit value key of the 64 lane maxima is a threshold that the
//           piece's top k all reach; only the 8-element groups whose maximum reaches it are listed, and only
//           their elements get order keys, which are ranked by counting); the k keys are written in rank order.
// Kernel 1 (k > 32): one workgroup of four waves per 8192 elements (four pieces): the pieces' sums as above,
//           and the top k of the 8192 elements (per-thread sorted lists, merged per wave, then per block).
// Kernel 2: one wave per row: combines the piece sums and merges the sorted candidate lists, writes
//           log-probs / ids.
#include <algorithm>
#include <atomic>

#include "mfd_common.h"
#include "exp_bf16_table.h"

#define MFD_LZ_PIECE 2048

namespace {

constexpr int PIECE = MFD_LZ_PIECE;  // log Z piece: one wave, 32 elements per lane
constexpr int CHUNK = 4 * PIECE;     // top-k unit of the k > 32 kernel (one workgroup of four waves)
constexpr int NT = 256;
constexpr int PER = CHUNK / NT;      // 32 elements per thread
constexpr int FINAL_STAGE = 4096;    // candidates per row staged in LDS by the k <= 32 merge (32 KB)
constexpr int KMAX = 256;            // a thread holds 32 elements: its 32-entry list keeps all of them for k > 32

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

// ---- the e^x table ------------------------------------------------------------------------------------
constexpr int ETAB = MFD_EXP_BF16_TABLE_SIZE;
__device__ const uint32_t exp_tab_g[ETAB] = {MFD_EXP_BF16_TABLE_INIT};
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Byte offsets (4 idx) into the table of the two bf16 values of a packed pair, in the two 16-bit halves:
// idx = min(max(rotl16(b, 1) - 0x6600, 0), 8191); v_pk_lshlrev_b16 / v_pk_lshrrev_b16 / v_pk_sub_u16 clamp /
// v_pk_min_u16, six operations for two elements.
__device__ __forceinline__ uint32_t etab_offsets(uint32_t pair) {
  const u16x2 b = __builtin_bit_cast(u16x2, pair);
  const u16x2 r = (b << (u16x2){1, 1}) | (b >> (u16x2){15, 15});
  u16x2 i = __builtin_elementwise_sub_sat(r, (u16x2){0x6600, 0x6600});
  i = __builtin_elementwise_min(i, (u16x2){ETAB - 1, ETAB - 1});
  return __builtin_bit_cast(uint32_t, (u16x2)(i << (u16x2){2, 2}));
}
__device__ __forceinline__ float etab_at(const float* etab, uint32_t byte_off) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(etab) + byte_off);
}

// One direct-to-LDS load (global_load_lds_dwordx4): lane l's 16 bytes at base + off land at LDS byte address
// lds_byte + 16 l (base and lds_byte wave-uniform). Waited for with s_waitcnt vmcnt(0) before the barrier that
// publishes the table.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds_byte) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds_byte);
  const uint64_t bb = (uint64_t)(uintptr_t)base;
  const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(bb >> 32)) << 32) |
                      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)bb);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(off), "s"(bs) : "memory", "m0");
}
// The table into LDS by the nwaves waves of a workgroup, 1 KB per load.
__device__ __forceinline__ void etab_stage(float* etab, int nwaves) {
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)etab;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int piece = w; piece < ETAB * 4 / 1024; piece += nwaves) {
    const uint32_t off = (uint32_t)piece * 1024u;
    dma16(exp_tab_g, off + 16u * lane, lds0 + off);
  }
}

// Lane sum of one piece: the lane's 32 elements raw[j][e] (piece element 512 j + 8 lane + e) in (j, e) order,
// against the piece maximum m. Elements at piece positions >= nvalid are past the row end: -inf in raw,
// contributing nothing. The polynomial path (m outside the table's range, rare) reads the elements again
// from psrc, the piece's first element.
__device__ __forceinline__ float piece_lane_sum(const u16x8 (&raw)[4], float m, const uint16_t* psrc, int nvalid,
                                                const float* etab) {
#pragma clang fp contract(off)
  float s = 0.f;
  if (m >= -60.0f && m < 64.0f) {
    // -m is a bf16 value too: its bits are m's upper half with the sign flipped
    const uint32_t mneg = ((__float_as_uint(m) >> 16) ^ 0x8000u) * 0x10001u;
    const float C = etab_at(etab, etab_offsets(mneg) & 0xFFFFu);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 u = __builtin_bit_cast(u32x4, raw[j]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t off = etab_offsets(u[q]);
        s = __builtin_fmaf(etab_at(etab, off & 0xFFFFu), C, s);
        s = __builtin_fmaf(etab_at(etab, off >> 16), C, s);
      }
    }
  } else if (m != -INFINITY) {
    const int l8 = 8 * (int)(threadIdx.x & 63);
#pragma unroll 1
    for (int j = 0; j < 4; ++j)
#pragma unroll 1
      for (int e = 0; e < 8; ++e) {
        const int idx = 512 * j + l8 + e;
        float t = 0.0f;
        if (idx < nvalid) {
          float d = bf2f(psrc[idx]) - m;
          d = d > -80.0f ? d : -80.0f;
          t = exp_det(d);
        }
        s = s + t;
      }
  }
  return s;
}

// Sum over the wave, pairwise over lane distances 32, 16, 8, 4, 2, 1: every lane ends with the same value.
__device__ __forceinline__ float wave_sum_tree(float v) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1)
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ d) << 2, __builtin_bit_cast(int, v)));
  return v;
}

// ---- keys and wave reductions -------------------------------------------------------------------------
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
// wave maximum of a 64-bit value (uniform result), the same way
__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t v) {
  auto step = [&](uint64_t o) { v = o > v ? o : v; };
  step(((uint64_t)row_ror32<1>((uint32_t)(v >> 32)) << 32) | row_ror32<1>((uint32_t)v));
  step(((uint64_t)row_ror32<2>((uint32_t)(v >> 32)) << 32) | row_ror32<2>((uint32_t)v));
  step(((uint64_t)row_ror32<4>((uint32_t)(v >> 32)) << 32) | row_ror32<4>((uint32_t)v));
  step(((uint64_t)row_ror32<8>((uint32_t)(v >> 32)) << 32) | row_ror32<8>((uint32_t)v));
  uint64_t best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t x = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((uint32_t)(v >> 32), 16 * r) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((uint32_t)v, 16 * r);
    best = x > best ? x : best;
  }
  return best;
}

// The k-th largest of the 64 lane values v < 2^BITS (0 = no value): the largest t with #{lanes: v >= t} >= k,
// found bit by bit from the top with ballots; 0 when fewer than k lanes hold a value. Wave-uniform.
template <int BITS = 32>
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t v, int k) {
  uint32_t t = 0;
#pragma unroll
  for (int bit = BITS - 1; bit >= 0; --bit) {
    const uint32_t c = t | (1u << bit);
    if (__builtin_popcountll(__builtin_amdgcn_ballot_w64(v >= c)) >= k) t = c;
  }
  return t;
}
// the same for 32-bit values in two 16-bit halves: the low halves only decide among the lanes tied at the
// boundary, and only when more of them are tied than are still needed
__device__ __forceinline__ uint32_t wave_kth_largest32s(uint32_t v, int k) {
  const uint32_t hi = v >> 16;
  const uint32_t th = wave_kth_largest<16>(hi, k);
  const int above = __builtin_popcountll(__builtin_amdgcn_ballot_w64(hi > th));
  const int tied = __builtin_popcountll(__builtin_amdgcn_ballot_w64(hi == th));
  const int need = k - above;
  uint32_t tl = 0;
  if (tied > need) tl = wave_kth_largest<16>(hi == th ? (v & 0xFFFFu) : 0u, need);
  return (th << 16) | tl;
}
// the same for 64-bit values in two 32-bit halves
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

// Piece keys are 32-bit: the upper half is the order key of the bf16 value (the upper 16 bits of
// float_order_key of the widened value; its lower 16 bits are 0 for positive and 0xFFFF for negative values,
// so nothing is lost), the lower half is 0xFFFF minus the element's index within the piece. Larger key =
// larger value, then smaller token id; keys are unique within a piece and never 0 (0 marks an empty lane).
__device__ __forceinline__ uint32_t piece_key(uint16_t raw, int local_idx) {
  const uint32_t b = __float_as_uint(bf2f(raw) + 0.0f);
  const uint32_t flip = (uint32_t)((int32_t)b >> 31) | 0x80000000u;
  return ((b ^ flip) & 0xFFFF0000u) | (uint32_t)(0xFFFF - local_idx);
}
// the 64-bit candidate key (cand_key) of a piece key, the piece starting at row element c0
__device__ __forceinline__ uint64_t global_key(uint32_t ck, int64_t c0) {
  const uint32_t hi = (ck & 0xFFFF0000u) | ((ck & 0x80000000u) ? 0u : 0xFFFFu);
  const int64_t idx = c0 + (0xFFFF - (int)(ck & 0xFFFFu));
  return ((uint64_t)hi << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}
// 16-bit order key of a widened bf16 value (larger value -> larger key; -0 counts as +0)
__device__ __forceinline__ uint32_t key16(float x) { return float_order_key(x + 0.0f) >> 16; }
// the smallest widened bf16 value whose key16 is t
__device__ __forceinline__ float key16_value(uint32_t t) {
  return __uint_as_float(((t & 0x8000u) ? (t & 0x7FFFu) : (~t & 0xFFFFu)) << 16);
}
// Number of the n keys in buf (LDS, 16-byte aligned, zero-padded to a multiple of 4) larger than v; every lane
// reads the same addresses (LDS broadcast).
__device__ __forceinline__ int count_greater(uint32_t v, const uint32_t* buf, int n) {
  int c = 0;
  for (int j = 0; j < n; j += 4) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(buf + j);
    c += (x[0] > v ? 1 : 0) + (x[1] > v ? 1 : 0) + (x[2] > v ? 1 : 0) + (x[3] > v ? 1 : 0);
  }
  return c;
}

struct FinalArgs {
  int rows, k;
  int npieces;         // (m, S) pairs per row
  int nlists;          // candidate lists of k keys per row
  const float* ws_m;
  const double* ws_s;
  const uint64_t* ws_cand;
  float* out_logp;     // [rows, k]
  void* out_ids;       // [rows, k] int32 or int64
  int ids_int64;
  float* out_logz;     // [rows] or null
  const int32_t* vocab_ids;  // [V] token id of each logit column, or null (column = token id)
};

struct ChunkArgs {
  const uint16_t* logits;
  int64_t row_stride;
  int rows, V, k;
  int npieces;        // pieces of PIECE elements per row
  int nchunks;        // chunks of CHUNK elements per row (the k > 32 kernel)
  float* ws_m;        // [rows * npieces]
  double* ws_s;       // [rows * npieces]
  uint64_t* ws_cand;  // [rows * npieces * k] (k <= 32) or [rows * nchunks * k] (k > 32)
};

// ---- kernel 1, k > 32 -----------------------------------------------------------------------------------
// One workgroup per (row, chunk of 8192 elements); wave w holds piece 4 chunk + w (its elements
// 512 j + 8 lane + e of the piece, raw[j][e]) and writes that piece's maximum and sum.
template <int KT>
__global__ __launch_bounds__(NT) void topk_logz_chunk_kernel(ChunkArgs a) {
  __shared__ uint64_t wcand[NT / 64][KMAX];
  __shared__ __attribute__((aligned(16))) float etab[ETAB];
  static_assert(NT == 256, "four pieces per chunk");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int row = blockIdx.x / a.nchunks;
  const int chunk = blockIdx.x % a.nchunks;
  const int piece = 4 * chunk + w;
  const int64_t p0 = (int64_t)piece * PIECE;
  const uint16_t* src = a.logits + (int64_t)row * a.row_stride;
  etab_stage(etab, NT / 64);

  // element (j, e) of this thread: index p0 + 512 j + 8 lane + e (increasing with (j, e))
  u16x8 raw[PER / 8];
#pragma unroll
  for (int j = 0; j < PER / 8; ++j) {
    const int64_t i0 = p0 + 512 * j + 8 * lane;
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
      const int64_t idx = p0 + 512 * j + 8 * lane + e;
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
  const float m = wave_max_dpp(mx);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's part of the table has landed
  __syncthreads();
  const int nvalid = (int)std::max<int64_t>(0, std::min<int64_t>((int64_t)PIECE, (int64_t)a.V - p0));
  const float ssum = wave_sum_tree(piece_lane_sum(raw, m, src + p0, nvalid, etab));
  if (lane == 0 && piece < a.npieces) {
    const int64_t ps = (int64_t)row * a.npieces + piece;
    a.ws_m[ps] = m;
    a.ws_s[ps] = (double)ssum;
  }
  // per-wave top-k, then the first wave merges the 4 wave lists
  wave_topk<KT>(list, a.k, wcand[w]);
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
  }
}

// ---- kernel 1, k <= 32 ----------------------------------------------------------------------------------
// One wave per piece, PW waves per workgroup sharing the table; a wave takes pieces (blockIdx.x * PW + wave) +
// i * gridDim.x * PW (piece id = row * npieces + piece). t_w, the k-th largest 16-bit value key of the 64 lane
// maxima, is reached by the piece's top k (k lanes reach it); the 8-element groups whose maximum reaches t_w
// are listed in LDS; the 32-bit keys of their elements with value keys >= t_w are formed one per lane (at most
// 8 listed groups; otherwise a running top k in 64-lane passes) and ranked by counting. Without ties at t_w
// fewer than 4 (k - 1) + 4 groups are listed, typically about k; with many ties up to all 256 (slower, still
// exact).
constexpr int PW = 16;  // waves per workgroup
// the row merge of kernel 2 for k <= 8 and at most 128 lists, by one wave (defined with kernel 2)
__device__ void final_row_fast(const FinalArgs& a, int row, double* terms);
// ROW: one workgroup per row of at most PW pieces (wave w takes piece w), and the workgroup's wave 0 merges
// the row once its pieces are written (no second kernel); otherwise kernel 2 merges
template <int KS, bool ROW>
__global__ __launch_bounds__(PW * 64) __attribute__((amdgpu_waves_per_eu(ROW ? 4 : 8))) void topk_piece_kernel(
    ChunkArgs a, FinalArgs f) {
  constexpr int CAPR = 8;  // listed groups whose raw values are staged in LDS (one 64-lane pass)
  __shared__ __attribute__((aligned(16))) float etab[ETAB];
  __shared__ uint16_t gfirst[PW][256];   // piece index of each listed group's first element
  __shared__ u16x8 graw[PW][CAPR];       // raw values of the first CAPR listed groups
  __shared__ __attribute__((aligned(16))) uint32_t keep_buf[PW][64];
  const int lane = threadIdx.x & 63;
  // the wave index in a scalar register: as a vector value it makes the per-wave LDS bases vector values too,
  // and at the 64-VGPR budget of eight waves per SIMD four of them spilled (scratch reloads on every piece)
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int k = a.k;
  const int total = a.rows * a.npieces;
  etab_stage(etab, PW);
  bool staged = false;  // every wave passes the one barrier that publishes the table exactly once
  const int pid0 = ROW ? (w < a.npieces ? (int)blockIdx.x * a.npieces + w : total) : (int)blockIdx.x * PW + w;
  const int pstep = ROW ? total : (int)gridDim.x * PW;
  for (int pid = pid0; pid < total; pid += pstep) {
    const int row = pid / a.npieces;
    const int64_t p0 = (int64_t)(pid - row * a.npieces) * PIECE;
    const uint16_t* psrc = a.logits + (int64_t)row * a.row_stride + p0;
    const int nvalid = (int)std::min<int64_t>((int64_t)PIECE, (int64_t)a.V - p0);
    // group j: piece elements 512 j + 8 lane + e; past the row end they read as -inf
    u16x8 raw[4];
    if (nvalid == PIECE) {
#pragma unroll
      for (int j = 0; j < 4; ++j) raw[j] = *reinterpret_cast<const u16x8*>(psrc + 512 * j + 8 * lane);
    } else {
      // the row's last piece: a group starting before the row end is read whole (the buffer holds
      // rows * row_stride elements, row_stride a multiple of 8), its elements past the end set to -inf
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i0 = 512 * j + 8 * lane;
        u16x8 x = {0xFF80u, 0xFF80u, 0xFF80u, 0xFF80u, 0xFF80u, 0xFF80u, 0xFF80u, 0xFF80u};
        if (i0 < nvalid) x = *reinterpret_cast<const u16x8*>(psrc + i0);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (i0 + e < nvalid) ? x[e] : (uint16_t)0xFF80u;
        raw[j] = x;
      }
    }
    // group maxima (widened floats), the lane maximum, the piece maximum and the threshold
    float gm[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 u = __builtin_bit_cast(u32x4, raw[j]);
      float x = -INFINITY;
#pragma unroll
      for (int q = 0; q < 4; ++q) x = fmaxf(x, fmaxf(__uint_as_float(u[q] << 16), __uint_as_float(u[q] & 0xFFFF0000u)));
      gm[j] = x;
    }
    const float lmax = fmaxf(fmaxf(gm[0], gm[1]), fmaxf(gm[2], gm[3]));
    const uint32_t tw = wave_kth_largest<16>(key16(lmax), k);
    const float m = wave_max_dpp(lmax);
    const float tv = key16_value(tw);
    // list the groups that may hold candidates (ballot + lane rank)
    int ng = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool take = gm[j] >= tv;
      const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
      if (mk) {
        if (take) {
          const int pos = ng + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0));
          gfirst[w][pos] = (uint16_t)(512 * j + 8 * lane);
          if (pos < CAPR) graw[w][pos] = raw[j];
        }
        ng += __builtin_popcountll(mk);
      }
    }
    if (!staged) {
      __builtin_amdgcn_s_waitcnt(0);  // this wave's part of the table has landed
      __syncthreads();
      staged = true;
    }
    // S_c before the selection, so that the raw values are dead during it
    const float ssum = wave_sum_tree(piece_lane_sum(raw, m, psrc, nvalid, etab));
    __builtin_amdgcn_wave_barrier();
    // element i of the listed groups is group i / 8, element i % 8
    auto fetch = [&](int i) -> uint32_t {
      if (i >= 8 * ng) return 0u;
      const int g = i >> 3;
      const int idx = (int)gfirst[w][g] + (i & 7);
      if (idx >= nvalid) return 0u;
      const uint16_t r = g < CAPR ? graw[w][g][i & 7] : psrc[idx];
      const uint32_t key = piece_key(r, idx);
      return (key >> 16) >= tw ? key : 0u;
    };
    uint32_t v = fetch(lane);
    uint64_t live;
    if (ng <= CAPR) {
      live = __builtin_amdgcn_ballot_w64(v != 0u);
    } else {
      // running top k: lanes hold the kept keys (low lanes) and the next unseen candidates
      int next = 64;
      for (;;) {
        const uint32_t t = wave_kth_largest32s(v, k);
        live = __builtin_amdgcn_ballot_w64(v != 0u && v >= t);
        if (next >= 8 * ng) break;
        const int nk = __builtin_popcountll(live);
        if ((live >> lane) & 1ull)
          keep_buf[w][__builtin_amdgcn_mbcnt_hi((uint32_t)(live >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)live, 0))] = v;
        __builtin_amdgcn_wave_barrier();
        v = lane < nk ? keep_buf[w][lane] : fetch(next + lane - nk);
        __builtin_amdgcn_wave_barrier();
        next += 64 - nk;
      }
    }
    // rank of each kept key among the kept keys (compacted into LDS, zero-padded to a multiple of 4); the
    // piece's list is written in rank order, zeros after its last key
    const bool kept = (live >> lane) & 1ull;
    const int nl = __builtin_popcountll(live);
    __builtin_amdgcn_wave_barrier();
    if (kept) keep_buf[w][__builtin_amdgcn_mbcnt_hi((uint32_t)(live >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)live, 0))] = v;
    if (lane >= nl && lane < ((nl + 3) & ~3)) keep_buf[w][lane] = 0u;
    __builtin_amdgcn_wave_barrier();
    const int rank = kept ? count_greater(v, keep_buf[w], nl) : 64;
    uint64_t* out = a.ws_cand + (int64_t)pid * k;
    if (rank < k) out[rank] = global_key(v, p0);
    if (lane >= nl && lane < k) out[lane] = 0;
    if (lane == 0) {
      a.ws_m[pid] = m;
      a.ws_s[pid] = (double)ssum;
    }
  }
  if (!staged) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if constexpr (ROW) {
    __shared__ double fterms[PW];
    __syncthreads();  // the row's piece lists, maxima and sums are written (the barrier orders global memory
                      // within the workgroup)
    if (w == 0) final_row_fast(f, blockIdx.x, fterms);
  }
}

// ---- kernel 2 -------------------------------------------------------------------------------------------

constexpr int FINAL_CAND = 8192;  // candidates of one row staged in LDS by the k > 32 merge (nlists * k)

__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t hi = (uint32_t)(key >> 32);
  return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
}

// The (m, S) of the row's first 256 pieces, piece c in lane c % 64, entry c / 64 (loaded before they are needed).
struct PieceSums {
  float m[4];
  double s[4];
};
__device__ __forceinline__ PieceSums load_piece_sums(const FinalArgs& a, int row) {
  const int lane = threadIdx.x & 63;
  const int np = a.npieces;
  PieceSums p;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int c = lane + 64 * r;
    p.m[r] = c < np ? a.ws_m[(int64_t)row * np + c] : -INFINITY;
    p.s[r] = c < np ? a.ws_s[(int64_t)row * np + c] : 0.0;
  }
  return p;
}
// log Z of row `row` from its pieces' (m, S), formed by one wave: the terms S_c exp_det(m_c - m) in parallel,
// added in piece order by a chain of lane reads (pieces past 256 through LDS scratch `terms` of npieces
// doubles); wave-uniform result.
__device__ float row_logz(const FinalArgs& a, int row, const PieceSums& p, double* terms) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int np = a.npieces;
  const float* mc = a.ws_m + (int64_t)row * np;
  const double* sc = a.ws_s + (int64_t)row * np;
  float m = fmaxf(fmaxf(p.m[0], p.m[1]), fmaxf(p.m[2], p.m[3]));
  for (int c = lane + 256; c < np; c += 64) m = fmaxf(m, mc[c]);
  m = wave_max_dpp(m);
  if (m == -INFINITY) return -INFINITY;
  // a piece whose maximum is -inf adds +0, which leaves the non-negative sum unchanged
  auto term = [&](float mcc, double s) -> double {
    if (mcc == -INFINITY) return 0.0;
    float d = mcc - m;
    d = d > -80.0f ? d : -80.0f;
    return s * (double)exp_det(d);
  };
  // the terms go to LDS, then every lane adds them in piece order (two per 16-byte read, eight reads in flight)
  for (int r = 0; r < 4; ++r)
    if (lane + 64 * r < np) terms[lane + 64 * r] = term(p.m[r], p.s[r]);
  for (int c = lane + 256; c < np; c += 64) terms[c] = term(mc[c], sc[c]);
  const int np2 = (np + 1) & ~1;
  if (lane == 0 && np2 != np) terms[np] = 0.0;  // adding +0 leaves the non-negative sum unchanged
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  typedef double f64x2 __attribute__((ext_vector_type(2)));
  const f64x2* t2 = reinterpret_cast<const f64x2*>(terms);
  double z = 0.0;
  int c = 0;
  for (; c + 16 <= np2; c += 16) {
    f64x2 x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = t2[c / 2 + i];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      z = z + x[i][0];
      z = z + x[i][1];
    }
  }
  for (; c < np2; c += 2) {
    const f64x2 x = t2[c / 2];
    z = z + x[0];
    z = z + x[1];
  }
  return (float)((double)m + log_det(z));
}


// k <= 8, at most 128 lists: each lane's (up to two) lists in registers; k rounds of "the largest head wins, its
// list shifts up by one entry"; winner i is kept by lane i, and the k outputs are written together once log Z
// is known. One wave; `terms`: LDS scratch of npieces doubles.
__device__ void final_row_fast(const FinalArgs& a, int row, double* terms) {
  const int lane = threadIdx.x & 63;
  const int k = a.k;
  const int nls = a.nlists;
  const uint64_t* src = a.ws_cand + (int64_t)row * nls * k;
  const PieceSums ps = load_piece_sums(a, row);
  auto put = [&](int pos, uint64_t key, float logz) {
    const float x = key ? key_value(key) : -INFINITY;
    uint32_t idx = key ? 0xFFFFFFFFu - (uint32_t)key : 0u;
    if (key && a.vocab_ids) idx = (uint32_t)a.vocab_ids[idx];
    a.out_logp[(int64_t)row * k + pos] = x - logz;
    if (a.ids_int64)
      static_cast<int64_t*>(a.out_ids)[(int64_t)row * k + pos] = (int64_t)idx;
    else
      static_cast<int32_t*>(a.out_ids)[(int64_t)row * k + pos] = (int32_t)idx;
  };
  uint64_t l0[8], l1[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    l0[j] = (lane < nls && j < k) ? src[lane * k + j] : 0ull;
    l1[j] = (lane + 64 < nls && j < k) ? src[(lane + 64) * k + j] : 0ull;
  }
  uint64_t win = 0ull;
  for (int i = 0; i < k; ++i) {
    const uint64_t mine = l0[0] > l1[0] ? l0[0] : l1[0];
    const uint64_t best = wave_max_u64_dpp(mine);
    if (lane == i) win = best;
    if (best != 0ull && mine == best) {  // keys are unique (they contain the token id)
      if (l0[0] == best) {
#pragma unroll
        for (int j = 0; j < 7; ++j) l0[j] = l0[j + 1];
        l0[7] = 0ull;
      } else {
#pragma unroll
        for (int j = 0; j < 7; ++j) l1[j] = l1[j + 1];
        l1[7] = 0ull;
      }
    }
  }
  const float logz = row_logz(a, row, ps, terms);
  if (lane < k) put(lane, win, logz);
  if (lane == 0 && a.out_logz) a.out_logz[row] = logz;
}

// k > 32: one wave per row, k rounds of wave argmax over the row's candidates
__global__ __launch_bounds__(64) void topk_logz_final_kernel(FinalArgs a) {
  __shared__ uint64_t cand[FINAL_CAND];
  __shared__ double terms[FINAL_CAND / 4];
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const int n = a.nlists * a.k;
  const uint64_t* src = a.ws_cand + (int64_t)row * n;
  const PieceSums ps = load_piece_sums(a, row);
  for (int t = lane; t < n; t += 64) cand[t] = src[t];
  const float logz = row_logz(a, row, ps, terms);
  // keys are unique (they contain the token id), the winner is removed
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

// k <= 32: one wave per row. The row's top k are merged from the pieces' rank-ordered lists (up to 128 lists:
// two list heads per lane, k rounds of "the largest head is output and its list advances"), or, for more
// lists, kept over all candidates in 64-lane passes (64-bit keys) and then ranked.
__global__ __launch_bounds__(64) void topk_small_final_kernel(FinalArgs a) {
  extern __shared__ __align__(16) unsigned char fsm[];
  double* terms = reinterpret_cast<double*>(fsm);  // [npieces]
  uint64_t* keep_buf = reinterpret_cast<uint64_t*>(terms + a.npieces);  // [64]
  uint64_t* cand = keep_buf + 64;  // [nlists k] when nlists k <= FINAL_STAGE: the row's candidates
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const int k = a.k;
  const int nls = a.nlists;
  const int n = nls * k;
  const uint64_t* src = a.ws_cand + (int64_t)row * n;
  auto put = [&](int pos, uint64_t key, float logz) {
    const float x = key ? key_value(key) : -INFINITY;
    uint32_t idx = key ? 0xFFFFFFFFu - (uint32_t)key : 0u;
    if (key && a.vocab_ids) idx = (uint32_t)a.vocab_ids[idx];
    a.out_logp[(int64_t)row * k + pos] = x - logz;
    if (a.ids_int64)
      static_cast<int64_t*>(a.out_ids)[(int64_t)row * k + pos] = (int64_t)idx;
    else
      static_cast<int32_t*>(a.out_ids)[(int64_t)row * k + pos] = (int32_t)idx;
  };
  const PieceSums ps = load_piece_sums(a, row);
  if (nls <= 128 && k <= 8) {
    final_row_fast(a, row, terms);
    return;
  }
  // the candidates are staged in LDS (four loads per lane in flight at a time, while log Z is formed), so
  // that the merge below reads no global memory
  const bool staged = n <= FINAL_STAGE;
  if (staged) {
    for (int i0 = 0; i0 < n; i0 += 256) {
      uint64_t x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = (i0 + 64 * r + lane < n) ? src[i0 + 64 * r + lane] : 0ull;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (i0 + 64 * r + lane < n) cand[i0 + 64 * r + lane] = x[r];
    }
  }
  const float logz = row_logz(a, row, ps, terms);
  if (k == 0) {
    if (lane == 0 && a.out_logz) a.out_logz[row] = logz;
    return;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  const uint64_t* cs = staged ? cand : src;
  if (nls <= 128) {
    int h0 = 0, h1 = 0;
    const bool has0 = lane < nls, has1 = lane + 64 < nls;
    uint64_t c0 = has0 ? cs[lane * k] : 0ull;
    uint64_t c1 = has1 ? cs[(lane + 64) * k] : 0ull;
    for (int i = 0; i < k; ++i) {
      const uint64_t mine = c0 > c1 ? c0 : c1;
      const uint64_t best = wave_max_u64_dpp(mine);
      if (best != 0ull && mine == best) {  // keys are unique (they contain the token id)
        if (c0 == best) {
          ++h0;
          c0 = h0 < k ? cs[lane * k + h0] : 0ull;
        } else {
          ++h1;
          c1 = h1 < k ? cs[(lane + 64) * k + h1] : 0ull;
        }
      }
      if (lane == 0) put(i, best, logz);
    }
    if (lane == 0 && a.out_logz) a.out_logz[row] = logz;
    return;
  }
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
  if (keep) put(rank, v, logz);
  if (lane >= nk && lane < k) put(lane, 0ull, logz);
  if (lane == 0 && a.out_logz) a.out_logz[row] = logz;
}

}  // namespace

extern "C" int64_t mfd_topk_logz_workspace_bytes(int rows, int V, int k) {
  const int64_t npieces = ((int64_t)V + PIECE - 1) / PIECE;
  // per piece: m (4 bytes), S (8) and up to k candidate keys (the k > 32 kernel keeps k per 4 pieces)
  return (int64_t)rows * npieces * (4 + 8 + 8 * (int64_t)(k > 0 ? k : 1)) + 64;
}

static int topk_logz_impl(const uint16_t* logits, int rows, int V, int64_t row_stride, int k, float* out_logp,
                          void* out_ids, int ids_int64, float* out_logz, const int32_t* vocab_ids, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  if (rows < 0 || V < 1 || k < 0 || k > V)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_topk_logz: bad sizes rows=%d V=%d k=%d", rows, V, k);
  if (k > KMAX) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_topk_logz: k=%d > %d", k, KMAX);
  const int npieces = (V + PIECE - 1) / PIECE;
  const int nchunks = (V + CHUNK - 1) / CHUNK;
  const int kk = k > 0 ? k : 1;
  const int nlists = kk <= 32 ? npieces : nchunks;
  if ((int64_t)nlists * kk > FINAL_CAND)
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
  char* ws = static_cast<char*>(workspace);
  uint64_t* cand = reinterpret_cast<uint64_t*>(ws);
  double* s = reinterpret_cast<double*>(ws + (int64_t)rows * npieces * kk * 8);
  float* m = reinterpret_cast<float*>(ws + (int64_t)rows * npieces * (kk * 8 + 8));
  ChunkArgs ca{logits, row_stride, rows, V, kk, npieces, nchunks, m, s, cand};
  FinalArgs fa{rows, k, npieces, nlists, m, s, cand, out_logp, out_ids, ids_int64, out_logz, vocab_ids};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (kk <= 32) {
    // one wave per piece while that fits two workgroups per CU; beyond, the waves loop over pieces
    const int64_t total = (int64_t)rows * npieces;
    if (k > 0 && k <= 8 && npieces <= PW) {
      // rows of at most PW pieces: one workgroup per row, which also merges it
      hipLaunchKernelGGL((topk_piece_kernel<8, true>), dim3((unsigned)rows), dim3(PW * 64), 0, st, ca, fa);
      MFD_CHECK_LAUNCH();
      return MFD_OK;
    }
    const dim3 grid((unsigned)std::min<int64_t>((total + PW - 1) / PW, 2 * (int64_t)mfd_num_cus()));
    if (kk <= 8)
      hipLaunchKernelGGL((topk_piece_kernel<8, false>), grid, dim3(PW * 64), 0, st, ca, fa);
    else if (kk <= 16)
      hipLaunchKernelGGL((topk_piece_kernel<16, false>), grid, dim3(PW * 64), 0, st, ca, fa);
    else
      hipLaunchKernelGGL((topk_piece_kernel<32, false>), grid, dim3(PW * 64), 0, st, ca, fa);
    MFD_CHECK_LAUNCH();
    {
      const int rc = mfd_set_max_lds(reinterpret_cast<const void*>(&topk_small_final_kernel), 160 * 1024);
      if (rc != MFD_OK) return rc;
    }
    const int ncand = nlists * k;
    const size_t smem = (size_t)(npieces + 64 + (ncand <= FINAL_STAGE ? ncand : 0)) * sizeof(double);
    hipLaunchKernelGGL(topk_small_final_kernel, dim3(rows), dim3(64), smem, st, fa);
    MFD_CHECK_LAUNCH();
    return MFD_OK;
  }
  const dim3 grid((unsigned)((int64_t)rows * nchunks));
  // k > 32: a thread's 32-entry list keeps all of its elements
  hipLaunchKernelGGL(topk_logz_chunk_kernel<PER>, grid, dim3(NT), 0, st, ca);
  MFD_CHECK_LAUNCH();
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
