// Exact mixture-tree builder for gfx950: one wave per request runs the best-first expansion of the
// reference's C++ heap (inference/hf/tree_build_ext.py:48-62 MixEntry / MixGreater, :158-203 build_mixture;
// batched form inference/sglang/patches/sglang-v0.5.22-mfd.patch:1330-1407) node for node:
//   - key = -(float(logw) + prior[mode]) in fp32, logw accumulated in fp64 as (logw - lp[r]) + lp[r + 1]
//     for a sibling and logw + lp[d][0] for a child;
//   - pop order: key, then mode, parent, depth, rank ascending (entries are unique in (mode, parent, rank),
//     so the logw tie-break of the reference is never reached); packed into one 64-bit key
//     (order-preserving float bits | mode 4b | parent 12b | depth 6b | rank 10b) so "next pop" is a
//     64-bit minimum over the frontier;
//   - a prefix popped again by another mode reuses its node (lookup by (parent, token) over the node table);
//     the budget counts distinct nodes.
// The frontier lives in LDS (a popped slot is reused by its sibling, the child takes a new slot); every pop
// is a wave-wide minimum over the live slots. The request's top log-probs / ids are staged in LDS.
// Outputs: tree[b] = tokens, depths, parents of width budget + 1 (index 0 = root: token 0, depth 0,
// parent -1; tail entries 0, 0, -1), counts[b], and optionally the ancestor-or-self matrix anc8[b]
// ([budget + 1]^2 int8, row i = row of parent(i) plus i; inference/hf/tree_build_ext.py:101-110).
#include "mfd_common.h"

namespace {

constexpr int WAVE = 64;

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

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const int src = (((int)threadIdx.x & 63) ^ mask) << 2;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const uint64_t o = shfl_xor_u64(v, m);
    v = o < v ? o : v;
  }
  return v;
}
__device__ __forceinline__ uint32_t pack_fields(int mode, int parent, int depth, int rank) {
  return ((uint32_t)mode << 28) | ((uint32_t)parent << 16) | ((uint32_t)depth << 10) | (uint32_t)rank;
}
__device__ __forceinline__ uint64_t entry_key(float key, uint32_t fields) {
  return ((uint64_t)float_order_key(key + 0.0f) << 32) | fields;
}

// LDS layout (dynamic): frontier keys u64 [cap], logw f64 [cap], lp f32 [K L k], ids i32 [K L k],
// node parent i32 / token i32 / depth i32 [budget + 1]
__global__ __launch_bounds__(WAVE) void build_mixture_kernel(BuildArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char smem[];
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int nlp = a.K * a.L * a.k;
  uint64_t* fkey = reinterpret_cast<uint64_t*>(smem);
  double* flogw = reinterpret_cast<double*>(fkey + a.cap);
  float* slp = reinterpret_cast<float*>(flogw + a.cap);
  int32_t* sid = reinterpret_cast<int32_t*>(slp + nlp);
  int32_t* npar = sid + nlp;
  int32_t* ntok = npar + (a.budget + 1);
  int32_t* ndep = ntok + (a.budget + 1);

  const float* lpb = a.lp + (int64_t)b * nlp;
  for (int i = lane; i < nlp; i += WAVE) {
    slp[i] = lpb[i];
    sid[i] = a.ids_int64 ? (int32_t) static_cast<const int64_t*>(a.ids)[(int64_t)b * nlp + i]
                         : static_cast<const int32_t*>(a.ids)[(int64_t)b * nlp + i];
  }
  const float* prior = a.prior ? a.prior + (int64_t)b * a.K : nullptr;
  const uint64_t DEAD = ~(uint64_t)0;
  // seed: one entry per mode (rank 0 at depth 1 under the root)
  int tail = a.K;
  for (int m = lane; m < a.cap; m += WAVE) fkey[m] = DEAD;
  __builtin_amdgcn_wave_barrier();
  for (int m = lane; m < a.K; m += WAVE) {
    const double lw = (double)lpb[(int64_t)m * a.L * a.k];
    const float pr = prior ? prior[m] : 0.f;
    fkey[m] = entry_key(-((float)lw + pr), pack_fields(m, 0, 1, 0));
    flogw[m] = lw;
  }
  if (lane == 0) {
    npar[0] = -1;
    ntok[0] = 0;
    ndep[0] = 0;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();

  int count = 0;
  int alive = a.K;
  bool overflow = false;
  // every iteration consumes a frontier entry and at most cap entries are ever pushed: bounded loop
  for (int iter = 0; iter < a.cap && alive > 0 && count < a.budget; ++iter) {
    uint64_t mine = DEAD;
    int where = -1;
    for (int s = lane; s < tail; s += WAVE) {
      const uint64_t e = fkey[s];
      if (e < mine) {
        mine = e;
        where = s;
      }
    }
    const uint64_t best = wave_min_u64(mine);
    const uint64_t win = __builtin_amdgcn_ballot_w64(mine == best && where >= 0);
    const int src_lane = (int)__builtin_ctzll(win);
    const int slot = __builtin_amdgcn_readlane(where, src_lane);
    const double logw = flogw[slot];
    const uint32_t f = (uint32_t)best;
    const int mode = (int)(f >> 28);
    const int parent = (int)((f >> 16) & 0xFFF);
    const int depth = (int)((f >> 10) & 0x3F);
    const int rank = (int)(f & 0x3FF);
    const int base = (mode * a.L + depth - 1) * a.k;
    const int token = sid[base + rank];
    // node of (parent, token): scan the node table
    int found = -1;
    for (int j = lane + 1; j <= count; j += WAVE)
      if (npar[j] == parent && ntok[j] == token) found = j;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(found >= 0);
    int current;
    if (hit) {
      current = __builtin_amdgcn_readlane(found, (int)__builtin_ctzll(hit));
    } else {
      current = count + 1;
      if (lane == 0) {
        npar[current] = parent;
        ntok[current] = token;
        ndep[current] = depth;
      }
      ++count;
    }
    const float pr = prior ? prior[mode] : 0.f;
    // sibling (rank + 1) takes over the popped slot, or the slot dies
    if (rank + 1 < a.k) {
      const double lw = (logw - (double)slp[base + rank]) + (double)slp[base + rank + 1];
      if (lane == 0) {
        fkey[slot] = entry_key(-((float)lw + pr), pack_fields(mode, parent, depth, rank + 1));
        flogw[slot] = lw;
      }
    } else {
      if (lane == 0) fkey[slot] = DEAD;
      --alive;
    }
    // child (depth + 1, rank 0) of the node just reached
    if (depth < a.L) {
      if (tail < a.cap) {
        const double lw = logw + (double)slp[(mode * a.L + depth) * a.k];
        if (lane == 0) {
          fkey[tail] = entry_key(-((float)lw + pr), pack_fields(mode, current, depth + 1, 0));
          flogw[tail] = lw;
        }
        ++tail;
        ++alive;
      } else {
        overflow = true;
        break;
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
  }
  if (overflow && lane == 0 && a.err) atomicOr(a.err, 1);

  // outputs
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
    // row i: ancestors of i and i itself (walk up the parents); rows past count stay zero
    for (int i = lane; i < W; i += WAVE) {
      int8_t* row = vis + (int64_t)i * W;
      for (int j = 0; j < W; ++j) row[j] = 0;
      if (i <= count) {
        int cur = i;
        while (cur >= 0) {
          row[cur] = 1;
          cur = npar[cur];
        }
      }
    }
  }
}

}  // namespace

extern "C" int mfd_build_mixture_smem_bytes(int K, int L, int k, int budget, int* cap_out) {
  const int64_t cap = (int64_t)K + 2LL * K * budget + 2;
  const int64_t c = cap > 4096 ? 4096 : cap;
  if (cap_out) *cap_out = (int)c;
  return (int)(c * 16 + (int64_t)K * L * k * 8 + (int64_t)(budget + 1) * 12);
}

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
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&build_mixture_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return mfd_set_hip_error(e);
    attr_set = true;
  }
  BuildArgs a{top_logp, top_ids, ids_int64, log_prior, bs, K, L, k, budget, cap, tree_out, counts_out, anc8_out,
              err_flag};
  hipLaunchKernelGGL(build_mixture_kernel, dim3(bs), dim3(WAVE), smem, static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
