/* mfd_hip.h — C ABI of libmfd_hip.so, the MI355X (gfx950) hot path of multi-future drafting.
 *
 * Conventions
 *   - Every entry point returns 0 on success or a negative MFD_ERR_* code; mfd_last_error() gives the
 *     message of the calling thread's last failure. Nothing here throws or aborts.
 *   - All tensor pointers are device pointers (HIP global memory) unless stated otherwise, row-major and
 *     contiguous in the layout written next to each argument. bf16 tensors are passed as uint16_t.
 *   - Kernels are enqueued on `stream` (a hipStream_t, NULL = the null stream); no host synchronisation,
 *     no allocation, no host read of device data. Calls are safe inside HIP graph capture.
 *   - The library keeps no state besides a per-device properties cache and, for mfd_tree_gdn_noalloc, one static
 *     device scratch array per GPU (MFD_GDN_SCRATCH_BYTES).
 */
#ifndef MFD_HIP_H
#define MFD_HIP_H

#include <stddef.h>
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
#define MFD_DEVERR_BAD_CONTEXT 8     /* a tree context built for another request size or max_nodes */
#define MFD_DEVERR_BAD_WINDOW 16     /* a conv window or accepted-path index outside its request / tree */
#define MFD_DEVERR_INTERNAL 32       /* a workgroup-internal hand-over wait ran out: that workgroup's outputs are NaN */

#define MFD_GDN_HEAD_DIM 128
#define MFD_GDN_MAX_DEPTH 16  /* nodes on a root path, root included */
#define MFD_GDN_MAX_NODES 512 /* nodes per tree (trees above 128 nodes take the two-kernel large-tree path) */

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
 *   cu_nodes  [R + 1] int32 node offsets of the requests (non-decreasing, cu_nodes[R] <= N; entries past N are
 *             clamped to N); may be NULL when R == 1 (then n = N)
 *   max_nodes upper bound on any request's node count (<= MFD_GDN_MAX_NODES); <= 128 runs the fused
 *             one-kernel path, above that the large-tree path (Gram rows per root-path slot, then the
 *             path-local solve), which needs a workspace
 *   u, o      [N, H, 128] f32 outputs
 *   err_flag  optional int32 device word; MFD_DEVERR_* bits are OR-ed in when a request is rejected (a root
 *             path over MFD_GDN_MAX_DEPTH nodes, a parent that does not precede its child, more nodes than
 *             max_nodes); the rejected request's u and o rows are then set to NaN
 *   workspace device scratch of mfd_tree_gdn_workspace_bytes(R, N, HK, max_nodes, 0) bytes, 256-byte aligned
 *             (NULL allowed when that is 0, i.e. max_nodes <= 128)
 */
int64_t mfd_tree_gdn_workspace_bytes(int R, int N, int HK, int max_nodes, int has_ctx);
int mfd_tree_gdn(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum, const float* beta,
                 const float* s0, const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R, int N,
                 int HK, int H, int D, int max_nodes, float* u, float* o, int32_t* err_flag, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* Allocation-free form of mfd_tree_gdn. No counterpart in the reference: for callers that cannot allocate
 * (code under HIP graph capture, serving loops that forbid hipMalloc). Same arguments and results as
 * mfd_tree_gdn without the workspace: the large-tree path (max_nodes > 128) uses a static device array of
 * MFD_GDN_SCRATCH_BYTES per GPU instead, so the call allocates nothing. Calls whose workspace
 * (mfd_tree_gdn_workspace_bytes(R, N, HK, max_nodes, 0)) exceeds it fail with MFD_ERR_UNSUPPORTED. The stream
 * must belong to the current device. Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, or threads) race and must be serialised by the caller.
 */
#define MFD_GDN_SCRATCH_BYTES (16 << 20)
int mfd_tree_gdn_noalloc(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum, const float* beta,
                         const float* s0, const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R,
                         int N, int HK, int H, int D, int max_nodes, float* u, float* o, int32_t* err_flag,
                         void* stream);

/* Tree context (replaces TreeContext, inference/hf/qwen35_tree.py:33-53: the ancestor matrix anc / anc_f /
 * anc8 built once per verify round and handed to every layer). For every request: each node's root path and
 * depth (and, for max_nodes <= 128, its ancestor-or-self bit mask), in the layout the tree-GDN kernels load
 * straight into LDS. Build it once per tree with mfd_tree_context, then pass it to the tree-GDN call of every
 * layer.
 *   mfd_tree_ctx_bytes  size of the context buffer of R requests for this max_nodes (0 for bad arguments)
 *   parents / anc8 / cu_nodes / R / N as for mfd_tree_gdn; max_nodes in [1, MFD_GDN_MAX_NODES]
 *   ctx, ctx_bytes  device buffer of at least mfd_tree_ctx_bytes(R, max_nodes) bytes, 16-byte aligned (output)
 *   err_flag  optional; MFD_DEVERR_TOO_MANY_NODES / TOO_DEEP / NOT_TOPOLOGICAL bits of rejected trees (they
 *             are also recorded in the context, and mfd_tree_gdn_ctx then rejects those requests)
 */
size_t mfd_tree_ctx_bytes(int R, int max_nodes);
int mfd_tree_context(const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R, int N, int max_nodes,
                     void* ctx, int64_t ctx_bytes, int32_t* err_flag, void* stream);

/* mfd_tree_gdn with the tree given as a context from mfd_tree_context (built with the same cu_nodes and
 * max_nodes) instead of parents / anc8; same outputs. ctx_bytes must cover mfd_tree_ctx_bytes(R, max_nodes) (the
 * kernels read R whole blocks). A request whose context does not match (node count, max_nodes) gets
 * MFD_DEVERR_BAD_CONTEXT and NaN outputs. workspace: mfd_tree_gdn_workspace_bytes(R, N, HK, max_nodes, 1) bytes
 * (0 for max_nodes <= 128). */
int mfd_tree_gdn_ctx(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum, const float* beta,
                     const float* s0, const void* ctx, int64_t ctx_bytes, const int32_t* cu_nodes, int R, int N, int HK,
                     int H, int D, int max_nodes, float* u, float* o, int32_t* err_flag, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* Gates of the tree-GDN layer (inference/hf/qwen35_tree.py:77-79, the torch lines before tree_gdn):
 *   beta_i = sigmoid(b_i),  g_i = -exp(A_log) * softplus(a_i + dt_bias)  (softplus(x) = x for x > 20),
 *   G_i = sum over the ancestors-or-self j of i of g_j   (the reference's anc_f @ g)
 *   a_proj, b_proj  [N, H] rows of row stride ab_row_stride, bf16 (ab_bf16 = 1) or f32
 *   A_log, dt_bias  [H] f32
 *   parents / anc8 / cu_nodes as for mfd_tree_gdn (no depth limit here)
 *   g_cum, beta     [N, H] f32 outputs, the g_cum / beta inputs of mfd_tree_gdn
 *   err_flag        optional; MFD_DEVERR_NOT_TOPOLOGICAL when a parent does not precede its child
 */
int mfd_tree_gates(const void* a_proj, const void* b_proj, int ab_bf16, int64_t ab_row_stride, const float* A_log,
                   const float* dt_bias, const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R,
                   int N, int H, float* g_cum, float* beta, int32_t* err_flag, void* stream);

/* Conv windows of the tree nodes (replaces TreeContext.conv_index, inference/hf/qwen35_tree.py:39-52, built
 * there by host loops): row i = node i's window of KC inputs, oldest first, as request-local indices into
 * [conv state (KC columns) ; the request's nodes] — i, its parent, grandparent, ..., then above the root the
 * cached columns KC - 1, KC - 2, ...
 *   parents / cu_nodes / R / N as for mfd_tree_gdn;  KC in [1, 8]
 *   conv_index [N, KC] int32 output;  err_flag optional (MFD_DEVERR_NOT_TOPOLOGICAL)
 */
int mfd_conv_index(const int32_t* parents, const int32_t* cu_nodes, int R, int N, int KC, int32_t* conv_index,
                   int32_t* err_flag, void* stream);

/* Tree convolution and q / k / v preparation (replaces tree_prep(), inference/hf/tree_gdn_kernel.py:135-150,
 * kernel _tree_prep :29-56). Channels are q heads, k heads, v heads (D = 128 each, CD = (2 HK + H) D):
 *   y = bf16(silu(sum_t conv_w[c][t] * window_t(c))),  window_t(c) = conv_state[c][idx] if idx < KC
 *       else x[idx - KC][c], idx = conv_index[i][t];
 *   q = bf16(y * rsqrt(sum_head y^2 + 1e-6) * scale), k = bf16(y * rsqrt(sum_head y^2 + 1e-6)), v = y
 *   x           [N, CD] bf16 pre-conv projections, row stride x_stride (a multiple of 8, >= CD); x, conv_state,
 *               conv_w and the outputs 16-byte aligned
 *   conv_state  [R][CD][KC] bf16 cached inputs (oldest first), request stride conv_state_req_stride
 *   conv_index  [N, KC] int32 windows (mfd_conv_index);  conv_w [CD, KC] bf16
 *   cu_nodes / R / N as for mfd_tree_gdn;  KC in [1, 8];  scale: q scale (the reference uses D^-0.5)
 *   q_out, k_out [N, HK, 128], v_out [N, H, 128] bf16
 *   err_flag    optional; MFD_DEVERR_BAD_WINDOW for a window index outside [0, KC + request nodes)
 */
int mfd_tree_prep(const uint16_t* x, int64_t x_stride, const uint16_t* conv_state, int64_t conv_state_req_stride,
                  const int32_t* conv_index, const uint16_t* conv_w, const int32_t* cu_nodes, int R, int N, int HK,
                  int H, int D, int KC, float scale, uint16_t* q_out, uint16_t* k_out, uint16_t* v_out,
                  int32_t* err_flag, void* stream);

/* Commit of the accepted path (replaces the state update of commit(), inference/hf/qwen35_tree.py:122-148),
 * all L GDN layers of one request in one launch; a = path[p - 1], the deepest accepted node:
 *   state_l,h <- exp(G_l[a,h]) state_l,h + sum_{j in path} exp(G_l[a,h] - G_l[j,h]) k_l[j, h/(H/HK)] u_l[j,h]^T
 *   conv_l[c][t] <- conv_l[c][idx] (old column) if idx < KC else x_l[idx - KC][c],  idx = conv_index[a][t]
 *   state   [L][H][128][128] f32 (the [d_k, d_v] layout), updated in place; layer stride in elements
 *   u       [L][n][H][128] f32, k [L][n][HK][128] bf16, g_cum [L][n][H] f32: the verify pass's values
 *   path    [p] int32 device, the accepted node ids (root first), 1 <= p <= n
 *   conv    [L][CD][KC] bf16 updated in place, or NULL to leave the conv states alone; then x, conv_index
 *           are ignored. x [L][n][CD] bf16 (row stride x_row_stride), conv_index [n, KC] int32
 *   err_flag  optional; MFD_DEVERR_BAD_WINDOW for a path or window index out of range (nothing is written
 *             when the deepest node itself is out of range)
 */
int mfd_gdn_commit(float* state, int64_t state_layer_stride, const float* u, int64_t u_layer_stride,
                   const uint16_t* k, int64_t k_layer_stride, const float* g_cum, int64_t g_layer_stride,
                   const int32_t* path, int p, int L, int n, int HK, int H, int D, uint16_t* conv,
                   int64_t conv_layer_stride, const uint16_t* x, int64_t x_layer_stride, int64_t x_row_stride,
                   const int32_t* conv_index, int CD, int KC, int32_t* err_flag, void* stream);


/* ---------------------------------------------------------------- K-mode drafter attention
 * Replaces mode_block_attention() (inference/hf/mode_attention.py:120-150: _mode_attn_split + _mode_attn_merge)
 * and paged_mode_block_attention() (inference/sglang/patches/sglang-v0.5.22-mfd.patch:897-962: the paged
 * split / merge / fused kernels). Query (b, head, qi) of mode qi / L attends to the context keys of request b
 * and to the L block keys of its own mode (all of them, or only t' <= t when causal_in_block).
 *
 *   q           token t = b K L + qi, head h: q + t * q_st + h * q_sh (bf16, 128 contiguous elements)
 *   k_new/v_new this step's block keys of token t, KV head g: k_new + t * kn_st + g * kn_sh
 *   k_cache/... context key of slot s, KV head g: k_cache + s * kc_ss + g * kc_sh (may be NULL when every
 *               context is empty)
 *   slot_table  NULL: slot = position (flat layout). page_size == 1: slot = slot_table[row * table_stride + t]
 *               (SGLang req_to_token). page_size > 1: slot = slot_table[row * table_stride + t / page_size] *
 *               page_size + t % page_size (page table). row = req_idx ? req_idx[b] : b (device int64)
 *   ctx_lens    device int64 [bs], or NULL to use ctx_len_const for every request
 *   num_ctx_splits  >= 1; 1 = one pass, > 1 = context split in that many chunks, the block keys in a partial
 *               of their own, and a log-sum-exp merge of the num_ctx_splits + 1 partials
 *   out         token t, head h: out + t * o_st + h * o_sh (bf16)
 *   workspace   device scratch of mfd_mode_attn_workspace_bytes(...) bytes (NULL allowed when 0)
 * Requires D == 128 and num_modes * block_size <= 65536 (any num_modes: when K * L is not a multiple of 32
 * the last 32-query unit of a head is padded).
 */
int64_t mfd_mode_attn_workspace_bytes(int bs, int num_modes, int block_size, int H, int num_ctx_splits);
int mfd_mode_attn(const uint16_t* q, int64_t q_st, int64_t q_sh, const uint16_t* k_new, const uint16_t* v_new,
                  int64_t kn_st, int64_t kn_sh, int64_t vn_st, int64_t vn_sh, const uint16_t* k_cache,
                  const uint16_t* v_cache, int64_t kc_ss, int64_t kc_sh, int64_t vc_ss, int64_t vc_sh,
                  const int32_t* slot_table, int64_t table_stride, int page_size, const int64_t* req_idx,
                  const int64_t* ctx_lens, int ctx_len_const, int bs, int num_modes, int block_size, int H, int Hkv,
                  int D, float scale, int causal_in_block, int num_ctx_splits, uint16_t* out, int64_t o_st,
                  int64_t o_sh, float* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- logits step (top-k + log Z)
 * Replaces top_candidates() / row_logsumexp() (inference/hf/tree_logits.py:16-46) and the SGLang
 * row_logsumexp (P:1451-1482) together with the torch.topk they pair with. Per row of bf16 logits:
 * the k largest values (value descending, token id ascending) as log-probabilities value - log Z (fp32)
 * and their ids (int32, or int64 when ids_int64), and log Z (optional). log Z is computed in one fixed
 * order of IEEE operations over 2048-element pieces (a table of e^x over bf16 x, fp32 sums in a fixed
 * lane / wave order, piece terms combined in fp64), exactly reproducible on the CPU.
 * k = 0: log Z only. Rows must start 16-byte aligned (row_stride % 8 == 0), and the buffer must hold
 * rows * row_stride elements (the last row's tail is read in 16-byte units up to the next multiple of 8).
 * Requires k <= 256 and a row merge of at most 8192 candidates: ceil(V / 2048) * max(k, 1) <= 8192 for
 * k <= 32 (one candidate list per 2048-element piece), ceil(V / 8192) * k <= 8192 for k > 32 (one list per
 * 8192 elements); beyond that MFD_ERR_UNSUPPORTED. mfd_topk_logz_workspace_bytes(rows, V, k) =
 * rows * ceil(V / 2048) * (12 + 8 max(k, 1)) + 64 bytes.
 */
int64_t mfd_topk_logz_workspace_bytes(int rows, int V, int k);
int mfd_topk_logz(const uint16_t* logits, int rows, int V, int64_t row_stride, int k, float* out_logp,
                  void* out_ids, int ids_int64, float* out_logz, void* workspace, int64_t workspace_bytes,
                  void* stream);

/* mfd_topk_logz over a reduced draft vocabulary (the id map of DDTreeDraftTopK, P:1535-1538): logit column c is
 * token vocab_ids[c] ([V] int32, device), so the ids written are vocab_ids[column]; log Z and the log-probs are
 * over the V columns (renormalised over the subset, as the reference). */
int mfd_topk_logz_vocab(const uint16_t* logits, int rows, int V, int64_t row_stride, int k, float* out_logp,
                        void* out_ids, int ids_int64, float* out_logz, const int32_t* vocab_ids, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* mfd_topk_logz for float32 or float16 logits (dtype MFD_DTYPE_F32 / MFD_DTYPE_F16): the reference's
 * top_candidates / row_logsumexp (inference/hf/tree_logits.py:34-46) and P:1451-1482 take the logits in any float
 * dtype (torch.topk in that dtype, an fp32 logsumexp of the same values). Same outputs as mfd_topk_logz (top k by
 * value descending, ties by column ascending; vocab_ids optional, NULL = identity); log Z = M + log(sum e^(x - M))
 * in fp32 (M the row maximum), within a few fp32 ulps of an fp64 logsumexp. Rows 16-byte aligned, row_stride a
 * multiple of 4 (f32) / 8 (f16) elements; k <= 256; no workspace. */
#define MFD_DTYPE_F32 0
#define MFD_DTYPE_F16 1
int mfd_topk_logz_wide(const void* logits, int dtype, int rows, int V, int64_t row_stride, int k, float* out_logp,
                       void* out_ids, int ids_int64, float* out_logz, const int32_t* vocab_ids, void* stream);

/* ---------------------------------------------------------------- draft top-k head
 * mfd_draft_head_gemm: the LM-head product of DDTreeDraftTopK (P:1523-1532: logits = hidden @ weight^T over the
 * drafted rows; the reference runs it as a library GEMM through torch.matmul), hand-written for gfx950.
 *   hidden   drafted row m (bf16) at hidden + (m / rows_per_group) * group_stride + (m % rows_per_group) * row_stride
 *            elements, so the drafted rows of a [bs * K * L, H] draft output are read in place (hidden = base + H,
 *            rows_per_group = L - 1, row_stride = H, group_stride = L * H); 16-byte aligned rows
 *   weight   [N, K] bf16 row-major, 16-byte aligned
 *   out      [M, out_stride] bf16 logits, out_stride >= N and a multiple of 4, 8-byte aligned
 * fp32 accumulation in k order, outputs rounded to nearest even. K must be a multiple of 64; the weight is
 * streamed once per 128 drafted rows.
 */
int mfd_draft_head_gemm(const uint16_t* hidden, int64_t row_stride, int rows_per_group, int64_t group_stride,
                        const uint16_t* weight, int M, int N, int K, uint16_t* out, int64_t out_stride, void* stream);

/* The whole draft top-k head (DDTreeDraftTopK.__call__, P:1523-1538) in one call: mfd_draft_head_gemm into
 * logits [M, logits_stride] (logits_stride a multiple of 8, 16-byte aligned), then the logits step over it
 * (mfd_topk_logz, or mfd_topk_logz_vocab when vocab_ids is not NULL) with the same outputs, workspace and limits.
 */
int mfd_draft_topk_head(const uint16_t* hidden, int64_t row_stride, int rows_per_group, int64_t group_stride,
                        const uint16_t* weight, int M, int N, int K, uint16_t* logits, int64_t logits_stride, int k,
                        float* out_logp, void* out_ids, int ids_int64, float* out_logz, const int32_t* vocab_ids,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- exact mixture-tree builder
 * Replaces build_mixture() (inference/hf/tree_build_ext.py:158-203) and build_trees() / build_mixture_one()
 * (P:1330-1407), on the device: the budget distinct prefixes with the largest max_k [log pi_k + sum log q_k],
 * node for node in the reference's pop order.
 *   top_logp   [bs, K, L, k] f32;  top_ids [bs, K, L, k] int32 (int64 when ids_int64);  log_prior [bs, K]
 *              f32 or NULL (uniform)
 *   tree_out   [bs, 3, budget + 1] int64: tokens, depths, parents (index 0 = root: 0, 0, -1; tail 0, 0, -1)
 *   counts_out [bs] int64 node counts;  anc8_out [bs, budget + 1, budget + 1] int8 ancestor-or-self or NULL
 *   err_flag   optional int32; bit 1 set if a request's frontier exceeded the kernel's capacity
 * Limits: K <= 16, L <= 63, k <= 1023, budget <= 4095, and the request's candidates plus frontier must fit
 * in LDS (mfd_build_mixture_smem_bytes <= 160 KiB).
 */
int mfd_build_mixture_smem_bytes(int K, int L, int k, int budget, int* cap_out);
int mfd_build_mixture(const float* top_logp, const void* top_ids, int ids_int64, const float* log_prior, int bs,
                      int K, int L, int k, int budget, int64_t* tree_out, int64_t* counts_out, int8_t* anc8_out,
                      int32_t* err_flag, void* stream);


/* The same builders on the host, for inputs and outputs in host memory: build_trees() (P:1377-1407), which the
 * patch's synchronous path calls with CPU tensors every round (P:1431-1445, 2889-2897), and the HF host-tensor
 * build_mixture / build_single (inference/hf/tree_build_ext.py:118-234). The mixture heap of mfd_build_mixture, or
 * for K == 1 with single_mode_heap the DDTree heap of mfd_build_single (the SGLang build_trees' choice; the HF
 * mixture builder keeps the mixture heap for one mode). Same trees node for node as the device builders.
 *   top_logp [bs, K, L, k] f32, top_ids [bs, K, L, k] int32 (int64 when ids_int64), log_prior [bs, K] f32 or NULL
 *   (uniform); tree_out [bs, 3, budget + 1] int64, counts_out [bs] int64, anc8_out [bs, budget + 1, budget + 1]
 *   int8 ancestor-or-self or NULL - all host memory, layouts and tails as mfd_build_mixture
 * No GPU work and no limits beyond K, L, k <= 65535; runs on the calling thread. */
int mfd_build_trees_host(const float* top_logp, const void* top_ids, int ids_int64, const float* log_prior, int bs,
                         int K, int L, int k, int budget, int single_mode_heap, int64_t* tree_out, int64_t* counts_out,
                         int8_t* anc8_out);

/* ---------------------------------------------------------------- single-mode DDTree builder
 * Replaces build_single() (inference/hf/tree_build_ext.py:118-156) and build_single_one() (P:1295-1328), the
 * builder of one-mode trees (build_trees with num_modes == 1): the budget best prefixes by the fp64 sum of
 * log-probabilities, node for node in the reference's pop order (key -logw in fp64, ties by the rank tuple
 * compared as a Python tuple; logw updated as (logw - lp[r]) + lp[r + 1] for a sibling, logw + lp[d][0] for
 * a child).
 *   top_logp [bs, L, k] f32;  top_ids [bs, L, k] int32 (int64 when ids_int64)
 *   tree_out, counts_out, anc8_out, err_flag as for mfd_build_mixture
 * Limits: L <= 63, k <= 1023, budget <= 4095, and mfd_build_single_smem_bytes <= 160 KiB.
 */
int mfd_build_single_smem_bytes(int L, int k, int budget, int* cap_out);
int mfd_build_single(const float* top_logp, const void* top_ids, int ids_int64, int bs, int L, int k, int budget,
                     int64_t* tree_out, int64_t* counts_out, int8_t* anc8_out, int32_t* err_flag, void* stream);

/* ---------------------------------------------------------------- verify-side plumbing
 * Verify inputs of a batch of trees (replaces ddtree_verify_inputs, P:1625-1700, the device form of
 * compile_ddtree_tree, inference/hf/ddtree.py:317-357). For request b and node i < W:
 *   mask row i at mask_out + mask_offsets[b] + i (prefix_lens[b] + W): prefix_lens[b] ones, then the
 *     ancestor-or-self bits of i over the W tree columns (walk of at most max_depth + 1 steps)
 *   ids_out[b, i] = root_tokens[b] (i = 0) or tokens[b, i];  positions_out[b, i] = prefix_lens[b] + depths[b, i]
 *   tokens / depths / parents: rows of tree_stride elements (the [bs, 3, W] tree of mfd_build_mixture gives
 *   tree_stride = 3 W); all int64; mask_out uint8 (bool); err_flag optional (MFD_DEVERR_BAD_WINDOW for a parent
 *   outside the tree)
 */
int mfd_verify_inputs(const int64_t* root_tokens, const int64_t* prefix_lens, const int64_t* tokens,
                      const int64_t* depths, const int64_t* parents, int64_t tree_stride, const int64_t* mask_offsets,
                      int64_t* ids_out, int64_t* positions_out, uint8_t* mask_out, int bs, int W, int max_depth,
                      int32_t* err_flag, void* stream);

/* HF verify inputs of one tree in the caller's persistent buffers (replaces compile_ddtree_tree,
 * inference/hf/ddtree.py:317-357). n1 = nodes + 1 (the root first):
 *   first mask[i][prev_start + j] = 0 for i, j < prev_len (the previous round's tree block joins the prefix);
 *   then ids_out[i] = root_token[0] (i = 0) or tokens[i - 1]; positions_out[i] = start (+ depths[i - 1]);
 *   vis_out[i * vis_out_stride + j] = visibility[i][j]; mask[i][past + j] = visibility[i][j] ? 0 : mask_min
 *   for i, j < n1.
 *   root_token [1] int64 (device); tokens, depths [n1 - 1] int64; visibility [n1, n1] bool (uint8)
 *   mask       mask_rows x mask_cols elements of mask_elem_bytes (2: bf16 / fp16, 4: fp32), rows
 *              mask_row_stride elements apart; mask_min_bits = the bit pattern of finfo(dtype).min
 * Every written row and column is checked against mask_rows / mask_cols and vis_out_stride.
 */
int mfd_tree_mask(const int64_t* root_token, int64_t start, const int64_t* tokens, const int64_t* depths,
                  const uint8_t* visibility, int n1, int64_t past, void* mask, int mask_elem_bytes,
                  uint32_t mask_min_bits, int64_t mask_row_stride, int64_t mask_cols, int mask_rows, int64_t* ids_out,
                  int64_t* positions_out, uint8_t* vis_out, int64_t vis_out_stride, int64_t prev_start, int prev_len,
                  void* stream);

/* Accept walk and commit moves of a verified batch (replaces ddtree_follow, P:1706-1766; the HF Tree.follow,
 * inference/hf/tree_build_ext.py:70-83): from the root, repeatedly the highest column whose parent is the
 * current node and whose verify id is the target's token at the current node (posterior), at most L - 1 steps.
 *   posterior, verify_ids, window [bs, W] int64; parents rows of parent_stride; prefix_lens [bs] int64
 *   accept_len_out, commit_lens_out [bs] int32 (n, n + 1); bonus_out [bs] = posterior at the last node;
 *   out_tokens_out [bs, L] (accepted tokens, the bonus, zeros); new_seq_lens_out [bs] = prefix + n + 1;
 *   move_src_out / move_tgt_out [bs, L] = window[path[j]] / window[j] for j <= n, else 0;
 *   hidden_index_out [bs, L] = b W + path[j] (path[j] = 0 past n). L <= 64.
 */
int mfd_tree_follow(const int64_t* posterior, const int64_t* verify_ids, const int64_t* parents, int64_t parent_stride,
                    const int64_t* window, const int64_t* prefix_lens, int32_t* accept_len_out,
                    int32_t* commit_lens_out, int64_t* bonus_out, int64_t* out_tokens_out, int64_t* new_seq_lens_out,
                    int64_t* move_src_out, int64_t* move_tgt_out, int64_t* hidden_index_out, int bs, int W, int L,
                    void* stream);

/* KV moves of the accepted paths (replaces _ddtree_compact_kv_kernel / DDTreeKVCompactor, P:1769-1841, and the
 * appended-window compaction of compact_dynamic_cache, inference/hf/ddtree.py:385-436). For every buffer and
 * request b, row move_src[b, j] is copied to row move_tgt[b, j] when they differ; every source of a request is
 * read before any of its targets is written. A row is nseg segments of seg_bytes at seg_stride_bytes apart
 * (1 segment for a token-major pool slot; the heads of a head-major [H, S, D] cache), rows row_stride_bytes
 * apart; rows outside [0, max_row) are skipped and flagged (MFD_DEVERR_BAD_WINDOW).
 *   buf_ptrs [nbuf] device array of buffer base addresses; move_src / move_tgt [bs, L] int64, L <= 64;
 *   seg_bytes, row_stride_bytes, seg_stride_bytes multiples of 16, buffers 16-byte aligned
 */
int mfd_kv_move(const uint64_t* buf_ptrs, int nbuf, int64_t row_stride_bytes, int nseg, int64_t seg_stride_bytes,
                int seg_bytes, int64_t max_row, const int64_t* move_src, const int64_t* move_tgt, int bs, int L,
                int32_t* err_flag, void* stream);

/* Draft-block inputs and the verify window of a round (replaces ddtree_prepare / _ddtree_prepare_kernel,
 * P:1557-1625). For request b:
 *   block_ids_out[b, l] = bonus_tokens[b] (l = 0) or mask_token_id;  positions_out[b, l] = prefix_lens[b] + l
 *   window_out[b, w] = req_to_token[req_pool_indices[b] * req_to_token_stride + prefix_lens[b] + w]   (w < W)
 *   bonus_tokens, prefix_lens, req_pool_indices, req_to_token: int32 or int64, bit 0 / 1 / 2 / 3 of
 *   index_int64_flags set for int64; outputs int64 ([bs, L], [bs, L], [bs, W]).
 */
int mfd_draft_prepare(const void* bonus_tokens, const void* prefix_lens, const void* req_pool_indices,
                      const void* req_to_token, int64_t req_to_token_stride, int index_int64_flags,
                      int64_t mask_token_id, int64_t* block_ids_out, int64_t* positions_out, int64_t* window_out,
                      int bs, int L, int W, void* stream);

/* Multi-mode draft mask (replaces ddtree_mode_mask / _ddtree_mode_mask_kernel, P:1889-1937): for request b
 * and row r < K L, the bool row at mask_out + mask_offsets[b] + r (prefix_lens[b] + K L) is prefix_lens[b] ones,
 * then 1 on the L columns of row r's own mode block (r / L) and 0 elsewhere. K L <= 65535.
 */
int mfd_mode_mask(const int64_t* prefix_lens, const int64_t* mask_offsets, uint8_t* mask_out, int bs, int num_modes,
                  int block_size, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MFD_HIP_H */
