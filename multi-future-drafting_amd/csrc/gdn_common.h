// Device helpers shared by the tree-GDN kernels (fused small-tree kernel and the large-tree path).
#pragma once
#include "mfd_common.h"

namespace gdn {

constexpr int D = MFD_GDN_HEAD_DIM;       // 128
constexpr int MAXD = MFD_GDN_MAX_DEPTH;   // nodes on a root path
constexpr int FUSED_MAX_NODES = 128;      // the fused kernel's limit; larger trees take the large-tree path
constexpr uint32_t RSRC_WORD3 = 0x00020000u;  // raw (untyped) buffer access

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)RSRC_WORD3);
}

// 4 x 4 transpose within each quad of lanes: lane i of the quad holds row i (x[0..3]) and receives column i.
__device__ __forceinline__ f32x4 quad_transpose(f32x4 x, int lane) {
  const bool odd = (lane & 1) != 0, hi2 = (lane & 2) != 0;
  f32x4 z, y;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float send = odd ? x[2 * p] : x[2 * p + 1];
    const float got = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, false));
    z[2 * p] = odd ? got : x[2 * p];
    z[2 * p + 1] = odd ? x[2 * p + 1] : got;
  }
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float send = hi2 ? z[p] : z[p + 2];
    const float got = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0x4E, 0xF, 0xF, false));
    y[p] = hi2 ? got : z[p];
    y[p + 2] = hi2 ? z[p + 2] : got;
  }
  return y;
}

// 16-byte store of four fp32 values. The values go through VGPRs element by element (a vector stored straight from
// MFMA accumulators once held element 0 four times) and the whole offset sits in the VGPR operand, soffset 0 (a
// 16-byte buffer store with an SGPR soffset was not protected against a VALU write to its data registers right after
// issue: stores lost data).
__device__ __forceinline__ void store4(__amdgpu_buffer_rsrc_t rs, uint32_t off, float x0, float x1, float x2, float x3) {
  asm volatile("" : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3));
  const u32x4 v = {__builtin_bit_cast(uint32_t, x0), __builtin_bit_cast(uint32_t, x1), __builtin_bit_cast(uint32_t, x2),
                   __builtin_bit_cast(uint32_t, x3)};
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 0);
}

// One direct-to-LDS load (global_load_lds_dwordx4): lane l's 16 bytes at base + off land at LDS byte
// address lds_byte + 16 l (base and lds_byte wave-uniform). Inline asm, so the compiler does not count it
// among its own loads; the kernel waits for it explicitly.
__device__ __forceinline__ void dma16_s(const void* base, uint32_t off, uint32_t lds_byte) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds_byte);
  const uint64_t bb = (uint64_t)(uintptr_t)base;
  // readfirstlane returns a signed int: go through uint32_t so that the low half is not sign-extended
  const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(bb >> 32)) << 32) |
                      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)bb);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(off), "s"(bs) : "memory", "m0");
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS byte address of a shared-memory object (for direct-to-LDS loads)
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) T*)p;
}

// Parent of node i of a request: parents[ns + i], or (single tree given as an ancestor-or-self matrix)
// the largest-index strict ancestor, since ancestors precede their descendants.
__device__ __forceinline__ int parent_of(const int32_t* parents, const int8_t* anc8, int ns, int i, int n) {
  if (parents) return parents[ns + i];
  const int8_t* row = anc8 + (size_t)i * n;
  for (int j = i - 1; j >= 0; --j)
    if (row[j] != 0) return j;
  return -1;
}

// Node range of request r: [ns, ns + n). cu_nodes entries past N are clamped to N, so a malformed
// cu_nodes never makes a kernel touch rows outside the [N, ...] tensors.
__device__ __forceinline__ void request_range(const int32_t* cu_nodes, int r, int N, int& ns, int& n) {
  if (!cu_nodes) {
    ns = 0;
    n = N;
    return;
  }
  const int a = min(max(cu_nodes[r], 0), N);
  const int b = min(max(cu_nodes[r + 1], 0), N);
  ns = a;
  n = b > a ? b - a : 0;
}

// Workgroups of one rejected request and value head mark its outputs: u and o rows [ns, ns + n) of head h,
// value columns [c0, c0 + nc), set to NaN (a rejection is never silent).
__device__ __forceinline__ void nan_fill(float* u, float* o, int ns, int n, int H, int h, int c0, int nc, int tid,
                                         int nthreads) {
  const float qnan = __builtin_nanf("");
  const int per = nc;
  for (int x = tid; x < n * per; x += nthreads) {
    const size_t off = ((size_t)(ns + x / per) * H + h) * D + c0 + x % per;
    u[off] = qnan;
    o[off] = qnan;
  }
}

}  // namespace gdn

// Host launchers of the large-tree path (tree_gdn_large.hip), called by the entry points in tree_gdn.hip.
struct GdnLargeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* g_cum;
  const float* beta;
  const float* s0;
  const int32_t* cu_nodes;
  const uint8_t* ctx;   // large-tree contexts (one block per request)
  float* gram;          // [N][HK][2][16] workspace
  float* u;
  float* o;
  int32_t* err;
  int R, N, HK, H;
  // set by the launcher when the Gram chunks run inside the main kernel (one-launch form): the per-(request, key
  // head) hand-over words; null for the two-kernel form
  uint32_t* gsync = nullptr;
};
size_t gdn_large_ctx_block_bytes(int max_nodes);
int gdn_large_context(const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R, int N,
                      int max_nodes, uint8_t* ctx, int32_t* err, hipStream_t s);
int gdn_large_run(const GdnLargeArgs& a, int max_nodes, hipStream_t s);
