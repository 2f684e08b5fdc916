// Logits step for float32 / float16 draft logits (the bf16 rows take logits_topk.hip): per row the top-k (value
// descending, token id ascending) and their log-probabilities value - log Z, with log Z = M + log(sum e^(x - M)),
// M the row maximum, summed in fp32 in a fixed order.
//
// Reference semantics: inference/hf/tree_logits.py:34-46 and inference/sglang/patches/sglang-v0.5.22-mfd.patch:
// 1451-1482, 1535-1538: torch.topk on the logits in their own dtype and an fp32 logsumexp of the same values;
// float16 values widen to float32 exactly, so both dtypes are handled as float32 values.
//
// One workgroup of 512 threads per row, four passes over the row (L2-resident after the first):
//   A  row maximum, histogram of the top 11 bits of the elements' order keys
//   B  sum of e^(x - M) (thread t takes the 16-byte vectors t, t + 512, ... in order, then a fixed reduction
//      tree), histogram of key bits 20..10 among the elements whose top 11 bits are the k-th largest's
//   C  histogram of key bits 9..0 among the elements whose top 22 bits are the k-th largest's: the k-th largest
//      key T and how many elements equal to T the top k holds (the lowest-indexed ones)
//   D  the elements above T (in any order) and the first elements equal to T (in index order) into LDS, then a
//      bitonic sort on (key, -index)
// The order key of a value: its bits with the sign bit set for x >= 0 and all bits flipped for x < 0 (-0 counts
// as +0; a NaN above +inf, as torch.topk orders it).
#include "mfd_common.h"

namespace {

constexpr int WT = 512;      // threads per row
constexpr int NBIN = 2048;   // radix digits of 11 bits
constexpr int KMAXW = 256;   // top-k limit (the bf16 path's)

struct WideArgs {
  const void* logits;
  int64_t row_stride;  // elements
  int V, k;
  float* out_logp;
  void* out_ids;
  int ids_int64;
  float* out_logz;
  const int32_t* vocab_ids;
};

__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t u = __float_as_uint(x);
  if (u == 0x80000000u) u = 0u;
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// the VEC values of 16-byte vector i of a row, as float32 (elements at or past V: -inf, flagged invalid)
template <typename T>
__device__ __forceinline__ void load_vec(const T* src, int i, int V, float (&x)[16 / sizeof(T)]) {
  constexpr int VEC = 16 / sizeof(T);
  const uint4 raw = *reinterpret_cast<const uint4*>(src + (int64_t)i * VEC);
  if constexpr (sizeof(T) == 4) {
    x[0] = __uint_as_float(raw.x); x[1] = __uint_as_float(raw.y); x[2] = __uint_as_float(raw.z); x[3] = __uint_as_float(raw.w);
  } else {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e] & 0xFFFFu));
      x[2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e] >> 16));
    }
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e)
    if (i * VEC + e >= V) x[e] = -__builtin_inff();
}

// Block-wide reductions of one value per thread (fixed order: within a wave by xor distances 32 .. 1, then the
// eight wave results in wave order).
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int x = 1; x < WT / 64; ++x) r = fmaxf(r, red[x]);
  return r;
}
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int x = 1; x < WT / 64; ++x) r += red[x];
  return r;
}

// After a histogram pass: the digit d of the k-th largest among the counted elements (need = how many of them the
// top k still takes), and how many counted elements lie above it. Thread t owns bins 4t .. 4t + 3.
__device__ __forceinline__ void select_digit(const uint32_t* hist, uint32_t need, uint32_t* scan, int& digit,
                                             uint32_t& above) {
  const int t = threadIdx.x;
  const uint32_t c0 = hist[4 * t], c1 = hist[4 * t + 1], c2 = hist[4 * t + 2], c3 = hist[4 * t + 3];
  const uint32_t own = c0 + c1 + c2 + c3;
  // suffix sums over threads (bins above this thread's): scan from the top thread down
  __syncthreads();
  scan[t] = own;
  __syncthreads();
  for (int d = 1; d < WT; d <<= 1) {
    const uint32_t add = (t + d < WT) ? scan[t + d] : 0u;
    __syncthreads();
    scan[t] += add;
    __syncthreads();
  }
  const uint32_t above_me = scan[t] - own;  // counted elements in bins above 4t + 3
  __syncthreads();
  // the digit where the count from the top first reaches need: exactly one thread finds it
  const uint32_t cs[4] = {c0, c1, c2, c3};
  uint32_t acc = above_me;
#pragma unroll
  for (int b = 3; b >= 0; --b) {
    if (acc < need && acc + cs[b] >= need) {
      scan[WT] = (uint32_t)(4 * t + b);
      scan[WT + 1] = acc;
    }
    acc += cs[b];
  }
  __syncthreads();
  digit = (int)scan[WT];
  above = scan[WT + 1];
  __syncthreads();
}

template <typename T>
__global__ __launch_bounds__(WT) void topk_logz_wide_kernel(WideArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ uint32_t hist[NBIN];
  __shared__ uint32_t scan[WT + 2];
  __shared__ float red[WT / 64];
  __shared__ uint64_t cand[KMAXW];
  __shared__ uint32_t ngt, neq_base;
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const T* src = reinterpret_cast<const T*>(a.logits) + (int64_t)row * a.row_stride;
  const int V = a.V, k = a.k;
  const int nvec = (V + VEC - 1) / VEC;

  // ---- A: row maximum; histogram of key bits 31..21
  for (int b = tid; b < NBIN; b += WT) hist[b] = 0u;
  __syncthreads();
  float m = -__builtin_inff();
  for (int i = tid; i < nvec; i += WT) {
    float x[VEC];
    load_vec<T>(src, i, V, x);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      m = fmaxf(m, x[e]);  // a NaN is dropped here; it shows in the sum below
      if (k > 0 && i * VEC + e < V) atomicAdd(&hist[order_key(x[e]) >> 21], 1u);
    }
  }
  const float M = block_max(m, red);

  int d0 = 0, d1 = 0, d2 = 0;
  uint32_t need = (uint32_t)k, above = 0;
  if (k > 0) {
    select_digit(hist, need, scan, d0, above);
    need -= above;
    for (int b = tid; b < NBIN; b += WT) hist[b] = 0u;
    __syncthreads();
  }
  // ---- B: sum of e^(x - M); histogram of key bits 20..10 under the prefix d0
  float s = 0.f;
  const bool finite_max = M > -__builtin_inff() && M < __builtin_inff();
  for (int i = tid; i < nvec; i += WT) {
    float x[VEC];
    load_vec<T>(src, i, V, x);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      if (i * VEC + e < V) {
        // (a NaN makes the sum NaN either way)
        s += finite_max ? expf(x[e] - M) : (x[e] == M ? 1.f : (x[e] != x[e] ? x[e] : 0.f));
        if (k > 0) {
          const uint32_t key = order_key(x[e]);
          if ((int)(key >> 21) == d0) atomicAdd(&hist[(key >> 10) & 2047u], 1u);
        }
      }
    }
  }
  const float S = block_sum(s, red);
  // log Z: M + log(sum); an all -inf row gives -inf, a row holding +inf gives +inf, a NaN gives NaN
  const float logz = finite_max ? M + logf(S) : (S != S ? S : M);

  if (k > 0) {
    select_digit(hist, need, scan, d1, above);
    need -= above;
    for (int b = tid; b < NBIN; b += WT) hist[b] = 0u;
    __syncthreads();
    // ---- C: histogram of key bits 9..0 under the prefix (d0, d1)
    const uint32_t pre22 = ((uint32_t)d0 << 11) | (uint32_t)d1;
    for (int i = tid; i < nvec; i += WT) {
      float x[VEC];
      load_vec<T>(src, i, V, x);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const uint32_t key = order_key(x[e]);
        if (i * VEC + e < V && (key >> 10) == pre22) atomicAdd(&hist[key & 1023u], 1u);
      }
    }
    __syncthreads();
    select_digit(hist, need, scan, d2, above);
    need -= above;  // elements equal to the threshold key that the top k takes (>= 1)
    const uint32_t thr = (pre22 << 10) | (uint32_t)d2;
    const uint32_t ngt_total = (uint32_t)k - need;

    // ---- D: the elements above thr (any order) into cand[0, ngt_total); the first `need` elements equal to thr,
    //      in index order, into cand[ngt_total, k). Candidates are (key, ~index) pairs.
    if (tid == 0) {
      ngt = 0u;
      neq_base = 0u;
    }
    __syncthreads();
    for (int i0 = 0; i0 < nvec; i0 += WT) {
      const int i = i0 + tid;
      float x[VEC];
      uint32_t keys[VEC];
      int eqc = 0;
      if (i < nvec) {
        load_vec<T>(src, i, V, x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const bool valid = i * VEC + e < V;
          keys[e] = order_key(x[e]);
          if (valid && keys[e] > thr) {
            const uint32_t slot = atomicAdd(&ngt, 1u);
            cand[slot] = ((uint64_t)keys[e] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(i * VEC + e));
          }
          eqc += (valid && keys[e] == thr) ? 1 : 0;
        }
      }
      // exclusive prefix of the equal counts over the threads (index order)
      scan[tid] = (uint32_t)eqc;
      __syncthreads();
      for (int d = 1; d < WT; d <<= 1) {
        const uint32_t add = tid >= d ? scan[tid - d] : 0u;
        __syncthreads();
        scan[tid] += add;
        __syncthreads();
      }
      const uint32_t base = neq_base;
      uint32_t r = base + scan[tid] - (uint32_t)eqc;
      const uint32_t chunk_total = scan[WT - 1];
      if (i < nvec && eqc > 0) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          if (i * VEC + e < V && keys[e] == thr) {
            if (r < need) cand[ngt_total + r] = ((uint64_t)thr << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(i * VEC + e));
            ++r;
          }
      }
      __syncthreads();
      if (tid == 0) neq_base = base + chunk_total;
      __syncthreads();
    }
    // ---- sort the k candidates descending (bitonic over the next power of two; padding sorts last)
    int kp = 1;
    while (kp < k) kp <<= 1;
    for (int j = tid + k; j < kp; j += WT) cand[j] = 0ull;
    __syncthreads();
    for (int size = 2; size <= kp; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int t = tid; t < kp / 2; t += WT) {
          const int lo = 2 * t - (t & (stride - 1));
          const int hi = lo + stride;
          const bool desc = ((lo & size) == 0);
          const uint64_t x = cand[lo], y = cand[hi];
          if ((x < y) == desc) {
            cand[lo] = y;
            cand[hi] = x;
          }
        }
        __syncthreads();
      }
    }
    for (int j = tid; j < k; j += WT) {
      const uint32_t idx = 0xFFFFFFFFu - (uint32_t)(cand[j] & 0xFFFFFFFFull);
      const float v = (float)src[idx];
      a.out_logp[(int64_t)row * k + j] = v - logz;
      const int32_t id = a.vocab_ids ? a.vocab_ids[idx] : (int32_t)idx;
      if (a.ids_int64)
        reinterpret_cast<int64_t*>(a.out_ids)[(int64_t)row * k + j] = id;
      else
        reinterpret_cast<int32_t*>(a.out_ids)[(int64_t)row * k + j] = id;
    }
  }
  if (tid == 0 && a.out_logz) a.out_logz[row] = logz;
}

}  // namespace

extern "C" int mfd_topk_logz_wide(const void* logits, int dtype, int rows, int V, int64_t row_stride, int k,
                                  float* out_logp, void* out_ids, int ids_int64, float* out_logz,
                                  const int32_t* vocab_ids, void* stream) {
  if (dtype != MFD_DTYPE_F32 && dtype != MFD_DTYPE_F16)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_topk_logz_wide: dtype %d is neither float32 nor float16", dtype);
  if (rows < 0 || V < 1 || k < 0 || k > V)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_topk_logz_wide: bad sizes rows=%d V=%d k=%d", rows, V, k);
  if (k > KMAXW) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_topk_logz_wide: k=%d > %d", k, KMAXW);
  const int vec = dtype == MFD_DTYPE_F32 ? 4 : 8;
  if (row_stride < V || (row_stride % vec) != 0 || (reinterpret_cast<uintptr_t>(logits) % 16) != 0)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_topk_logz_wide: rows must be 16-byte aligned (stride %lld)",
                         (long long)row_stride);
  if (rows == 0) return MFD_OK;
  if (!logits || (k > 0 && (!out_logp || !out_ids)) || (k == 0 && !out_logz))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_topk_logz_wide: null pointer");
  const WideArgs args{logits, row_stride, V, k, out_logp, out_ids, ids_int64, out_logz, vocab_ids};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MFD_DTYPE_F32)
    hipLaunchKernelGGL(topk_logz_wide_kernel<float>, dim3((unsigned)rows), dim3(WT), 0, st, args);
  else
    hipLaunchKernelGGL(topk_logz_wide_kernel<_Float16>, dim3((unsigned)rows), dim3(WT), 0, st, args);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
