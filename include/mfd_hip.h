/* mfd_hip.h — C ABI of libmfd_hip.so, the MI355X (gfx950) hot path of multi-future drafting.
 *
 * Conventions
 *   - Every entry point returns 0 on success or a negative MFD_ERR_* code; mfd_last_error() gives the
 *     message of the calling thread's last failure. Nothing here throws or aborts.
 *   - All tensor pointers are device pointers (HIP global memory) unless stated otherwise, row-major and
 *     contiguous in the layout written next to each argument. bf16 tensors are passed as uint16_t.
 *   - Kernels are enqueued on `stream` (a hipStream_t, NULL = the null stream); no host synchronisation,
 *     no allocation, no host read of device data. Calls are safe inside HIP graph capture.
 *   - The library keeps no state besides a per-device properties cache.
 */
#ifndef MFD_HIP_H
#define MFD_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MFD_OK 0
#define MFD_ERR_INVALID_ARG (-1)   /* bad shape, null pointer, size out of range */
#define MFD_ERR_UNSUPPORTED (-2)   /* valid but not supported by this build (e.g. head dim != 128) */
#define MFD_ERR_HIP (-3)           /* a HIP runtime call failed (launch error, ...) */

/* Device-side error bits written (atomic OR) into the optional `err_flag` argument. */
#define MFD_DEVERR_TOO_MANY_NODES 1  /* a request has more nodes than max_nodes / the kernel's limit */
#define MFD_DEVERR_TOO_DEEP 2        /* a root path is longer than MFD_GDN_MAX_DEPTH nodes */
#define MFD_DEVERR_NOT_TOPOLOGICAL 4 /* parents[i] >= i */

#define MFD_GDN_HEAD_DIM 128
#define MFD_GDN_MAX_DEPTH 16  /* nodes on a root path, root included */
#define MFD_GDN_MAX_NODES 128 /* nodes per tree */

const char* mfd_last_error(void);
int mfd_version(void);

/* ---------------------------------------------------------------- tree gated-delta-rule verify
 * Replaces tree_gdn() (inference/hf/tree_gdn_kernel.py:153-171: _tree_kkt + fla solve_tril + _tree_u)
 * and adds the ragged batch the reference lacks. For every node i of every request (nodes in
 * topological order, parents first; value head h reads key head h / (H / HK)):
 *   u_i + sum_{j strict anc i} beta_i e^{G_i-G_j} (k_i.k_j) u_j = beta_i (v_i - e^{G_i} S0^T k_i)
 *   o_i = e^{G_i} S0^T q_i + sum_{j anc-or-self i} e^{G_i-G_j} (q_i.k_j) u_j
 *
 *   q, k      [N, HK, 128] bf16 (q already scaled as the caller wants it; the reference scales in tree_prep)
 *   v         [N, H, 128]  bf16
 *   g_cum     [N, H] f32   G_i: log decay summed along the root path (node i included)
 *   beta      [N, H] f32
 *   s0        [R, H, 128, 128] f32, the committed state of each request in the [d_k, d_v] layout
 *   parents   [N] int32, request-local parent index, -1 for the root; may be NULL when anc8 is given
 *   anc8      [n, n] int8 ancestor-or-self matrix of a single tree (R == 1); used only when parents is NULL
 *   cu_nodes  [R + 1] int32 node offsets of the requests; may be NULL when R == 1 (then n = N)
 *   max_nodes upper bound on any request's node count (<= MFD_GDN_MAX_NODES), chooses the kernel variant
 *   u, o      [N, H, 128] f32 outputs
 *   err_flag  optional int32 device word; MFD_DEVERR_* bits are OR-ed in when a request is rejected
 *             (its outputs are then left unwritten)
 */
int mfd_tree_gdn(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum, const float* beta,
                 const float* s0, const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R, int N,
                 int HK, int H, int D, int max_nodes, float* u, float* o, int32_t* err_flag, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MFD_HIP_H */
