// Verify-side plumbing of a tree round for gfx950: the target's verify inputs built from the trees, the walk
// that accepts the verified path, and the KV moves that compact the accepted path.
//
//   tree mask (inference/hf/ddtree.py:317-357 compile_ddtree_tree, the HF form): one tree's verify ids and
//     positions and its block of the additive attention mask (0 where the builder's visibility matrix has the
//     key, finfo(dtype).min elsewhere) written into the caller's persistent buffers, after the previous
//     round's block is cleared to 0.
//   verify inputs (inference/sglang/patches/sglang-v0.5.22-mfd.patch:1625-1700 _ddtree_verify_inputs_kernel,
//     the device form of compile_ddtree_tree, inference/hf/ddtree.py:317-357): for request b and node i,
//     mask row i = [prefix ones | ancestor-or-self bits of i over the W tree columns] (flat, at
//     mask_offsets[b], row length prefix + W), ids[b, i] = root token (i = 0) or the node's token,
//     positions[b, i] = prefix + depth[i]. The ancestor walk takes at most max_depth + 1 steps.
//   follow (P:1706-1766 _ddtree_follow_kernel; inference/hf/tree_build_ext.py:70-83 Tree.follow): from the
//     root, the child whose token is the target's token at the current node (the highest such column),
//     for at most L - 1 steps; emits the accepted tokens plus the bonus, the path's hidden-row indices, and
//     the KV moves window[path[j]] -> window[j] of the accepted path (no-moves as 0 -> 0).
//   KV moves (P:1769-1841 _ddtree_compact_kv_kernel; inference/hf/ddtree.py:385-436 compaction of the
//     appended window): for every buffer, the rows src -> tgt of each request whose source differs from its
//     target; all sources of a request are read before any target is written (a target can be another
//     move's source).
//   draft prepare (P:1557-1625 _ddtree_prepare_kernel): per request, the draft block's ids (the bonus token,
//     then the mask token) and positions (prefix + l), and the verify window's cache slots
//     req_to_token[req_pool_indices[b], prefix + w] for w < W.
//   mode mask (P:1889-1937 _ddtree_mode_mask_kernel): row r of request b's multi-mode draft mask
//     [K * L, prefix + K * L] at mask_offsets[b] = [prefix ones | 1 on the L columns of row r's own mode block].
#include "mfd_common.h"

namespace {

constexpr int MAXL = 64;  // accepted-path length bound of the follow and move kernels

// Bytes [0, n) of row set to 1 by the workgroup's 256 threads: single bytes up to the first 16-byte boundary,
// then 16-byte stores, then the tail.
__device__ __forceinline__ void fill_ones(uint8_t* row, int64_t n, int tid) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(row);
  const int64_t lead = (int64_t)((16 - (addr & 15)) & 15);
  const int64_t head = lead < n ? lead : n;
  for (int64_t j = tid; j < head; j += 256) row[j] = 1;
  const int64_t nvec = (n - head) / 16;
  const uint4 ones = make_uint4(0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u);
  for (int64_t v = tid; v < nvec; v += 256) reinterpret_cast<uint4*>(row + head)[v] = ones;
  for (int64_t j = head + nvec * 16 + tid; j < n; j += 256) row[j] = 1;
}

// ---- verify inputs: one workgroup per (request, node)
struct VerifyArgs {
  const int64_t* root;
  const int64_t* prefix;
  const int64_t* tok;
  const int64_t* dep;
  const int64_t* par;
  int64_t tree_stride;
  const int64_t* mask_off;
  int64_t* ids;
  int64_t* pos;
  uint8_t* mask;
  int W, max_depth;
  int32_t* err;
};

__global__ __launch_bounds__(256) void verify_inputs_kernel(VerifyArgs a) {
  extern __shared__ uint8_t vis[];  // [W]
  const int b = blockIdx.x / a.W, i = blockIdx.x % a.W;
  const int tid = threadIdx.x;
  const int64_t prefix = a.prefix[b];
  const int64_t row_len = prefix + a.W;
  uint8_t* row = a.mask + a.mask_off[b] + (int64_t)i * row_len;
  for (int j = tid; j < a.W; j += 256) vis[j] = 0;
  __syncthreads();
  if (tid == 0) {
    const int64_t* par = a.par + (int64_t)b * a.tree_stride;
    int64_t anc = i;
    for (int s = 0; s <= a.max_depth && anc >= 0; ++s) {
      vis[anc] = 1;
      if (anc == 0) break;
      const int64_t nxt = par[anc];
      if (nxt >= a.W) {  // a parent outside the tree: stop, flagged
        if (a.err) atomicOr(a.err, MFD_DEVERR_BAD_WINDOW);
        break;
      }
      anc = nxt;
    }
    a.ids[(int64_t)b * a.W + i] = i == 0 ? a.root[b] : a.tok[(int64_t)b * a.tree_stride + i];
    a.pos[(int64_t)b * a.W + i] = prefix + a.dep[(int64_t)b * a.tree_stride + i];
  }
  fill_ones(row, prefix, tid);
  __syncthreads();
  for (int j = tid; j < a.W; j += 256) row[prefix + j] = vis[j];
}

// ---- draft prepare: one workgroup per request
struct PrepareArgs {
  const void* bonus;
  const void* prefix;
  const void* req_pool;
  const void* r2t;       // req_to_token [pool rows, r2t_stride]
  int64_t r2t_stride;
  int flags;             // bit 0/1/2/3: bonus / prefix / req_pool / req_to_token hold int64 (else int32)
  int64_t mask_token;
  int64_t* block_ids;    // [bs, L]
  int64_t* block_pos;    // [bs, L]
  int64_t* window;       // [bs, W]
  int L, W;
};

__device__ __forceinline__ int64_t load_index(const void* p, int64_t i, bool wide) {
  return wide ? static_cast<const int64_t*>(p)[i] : (int64_t) static_cast<const int32_t*>(p)[i];
}

__global__ __launch_bounds__(256) void draft_prepare_kernel(PrepareArgs a) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t prefix = load_index(a.prefix, b, a.flags & 2);
  for (int l = tid; l < a.L; l += 256) {
    a.block_ids[(int64_t)b * a.L + l] = l == 0 ? load_index(a.bonus, b, a.flags & 1) : a.mask_token;
    a.block_pos[(int64_t)b * a.L + l] = prefix + l;
  }
  const int64_t row = load_index(a.req_pool, b, a.flags & 4) * a.r2t_stride + prefix;
  for (int w = tid; w < a.W; w += 256) a.window[(int64_t)b * a.W + w] = load_index(a.r2t, row + w, a.flags & 8);
}

// ---- mode mask: one workgroup per (request, row)
__global__ __launch_bounds__(256) void mode_mask_kernel(const int64_t* prefix_lens, const int64_t* mask_off,
                                                        uint8_t* mask, int KL, int L) {
  const int b = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x;
  const int64_t prefix = prefix_lens[b];
  uint8_t* row = mask + mask_off[b] + (int64_t)r * (prefix + KL);
  fill_ones(row, prefix, tid);
  const int mode = r / L;
  for (int c = tid; c < KL; c += 256) row[prefix + c] = (c / L) == mode;
}

// ---- follow: one wave per request
struct FollowArgs {
  const int64_t* post;   // [bs, W]
  const int64_t* tok;    // verify ids [bs, W]
  const int64_t* par;    // [bs, parent_stride]
  int64_t par_stride;
  const int64_t* window; // [bs, W]
  const int64_t* prefix; // [bs]
  int32_t* accept_len;
  int32_t* commit_len;
  int64_t* bonus;
  int64_t* out_tokens;   // [bs, L]
  int64_t* new_seq;
  int64_t* mv_src;       // [bs, L]
  int64_t* mv_tgt;       // [bs, L]
  int64_t* hid_idx;      // [bs, L]
  int W, L;
};

__global__ __launch_bounds__(64) void tree_follow_kernel(FollowArgs a) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t* post = a.post + (int64_t)b * a.W;
  const int64_t* tok = a.tok + (int64_t)b * a.W;
  const int64_t* par = a.par + (int64_t)b * a.par_stride;
  int64_t path_l = 0, emit_l = 0;  // lane j holds path[j] and emitted[j]
  int64_t cur = 0;
  int n = 0;
  for (int step = 0; step < a.L - 1; ++step) {
    const int64_t t = post[cur];
    int best = -1;  // highest column whose parent is cur and whose token is t
    for (int c = lane; c < a.W; c += 64)
      if (par[c] == cur && tok[c] == t) best = c;
    // wave maximum of best
    int m = best;
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = max(m, __shfl_xor(m, s));
    if (m < 0) break;
    if (lane == n) emit_l = t;
    ++n;
    if (lane == n) path_l = m;
    cur = m;
  }
  const int64_t bon = post[cur];
  if (lane == n) emit_l = bon;
  const int64_t prefix = a.prefix[b];
  const bool live = lane <= n;
  if (lane < a.L) {
    const int64_t o = (int64_t)b * a.L + lane;
    a.out_tokens[o] = lane <= n ? emit_l : 0;
    a.hid_idx[o] = (int64_t)b * a.W + (live ? path_l : 0);
    a.mv_src[o] = live ? a.window[(int64_t)b * a.W + path_l] : 0;
    a.mv_tgt[o] = live ? a.window[(int64_t)b * a.W + lane] : 0;
  }
  if (lane == 0) {
    a.accept_len[b] = n;
    a.commit_len[b] = n + 1;
    a.bonus[b] = bon;
    a.new_seq[b] = prefix + n + 1;
  }
}

// ---- KV moves: one workgroup per (request, buffer, tile of the row)
struct MoveArgs {
  const uint64_t* bufs;  // [nbuf] base addresses
  int64_t row_stride;    // bytes between rows
  int nseg;              // segments per row (e.g. heads of a head-major layout)
  int64_t seg_stride;    // bytes between segments
  int seg_bytes;         // bytes per segment (a multiple of 16)
  const int64_t* src;    // [bs, L]
  const int64_t* tgt;    // [bs, L]
  int L, tiles_per_seg;
  int64_t max_row;       // rows are checked against [0, max_row)
  int32_t* err;
};

constexpr int TILE = 1024;  // bytes of a segment per workgroup pass (64 x 16)

__global__ __launch_bounds__(256) void kv_move_kernel(MoveArgs a) {
  __shared__ int64_t mv[2][MAXL];  // this request's moves (target -1: nothing to move)
  __shared__ int any;
  const int b = blockIdx.x;
  const int buf = blockIdx.y;
  const int seg = blockIdx.z / a.tiles_per_seg;
  const int tile = blockIdx.z % a.tiles_per_seg;
  const int tid = threadIdx.x;
  if (tid == 0) any = 0;
  __syncthreads();
  if (tid < a.L) {
    const int64_t s = a.src[(int64_t)b * a.L + tid], t = a.tgt[(int64_t)b * a.L + tid];
    bool ok = s != t;
    if (ok && (s < 0 || t < 0 || s >= a.max_row || t >= a.max_row)) {
      ok = false;
      if (blockIdx.y == 0 && blockIdx.z == 0 && a.err) atomicOr(a.err, MFD_DEVERR_BAD_WINDOW);
    }
    mv[0][tid] = s;
    mv[1][tid] = ok ? t : -1;
    if (ok) any = 1;
  }
  __syncthreads();
  if (!any) return;
  const int g = tid >> 6;      // moves g, g + 4, ...
  const int c = tid & 63;      // 16-byte chunk of the tile
  const int64_t off = (int64_t)tile * TILE + (int64_t)c * 16;
  const bool in_seg = off + 16 <= a.seg_bytes;
  uint8_t* base = reinterpret_cast<uint8_t*>(a.bufs[buf]) + (int64_t)seg * a.seg_stride + off;
  constexpr int PER = MAXL / 4;
  uint4 v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int j = g + 4 * q;
    if (j < a.L && mv[1][j] >= 0 && in_seg) v[q] = *reinterpret_cast<const uint4*>(base + mv[0][j] * a.row_stride);
  }
  __syncthreads();  // every source of this request's tile is read before any target is written
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int j = g + 4 * q;
    if (j < a.L && mv[1][j] >= 0 && in_seg) *reinterpret_cast<uint4*>(base + mv[1][j] * a.row_stride) = v[q];
  }
}

// ---- HF verify inputs of one tree (the additive-mask form): one workgroup per mask row
struct TreeMaskArgs {
  const int64_t* root;    // [1]
  int64_t start;          // position of the root
  const int64_t* tok;     // [n1 - 1] node tokens
  const int64_t* dep;     // [n1 - 1] node depths
  const uint8_t* vis;     // [n1, n1] ancestor-or-self (bool)
  int n1;
  int64_t past;           // first tree column of the mask
  uint8_t* mask;          // rows of mask_row_bytes
  int64_t mask_row_bytes;
  int esize;              // 2 or 4 bytes per mask element
  uint32_t min_bits;      // the element written where a key is not visible (finfo(dtype).min)
  int64_t* ids;
  int64_t* pos;
  uint8_t* vis_out;
  int64_t vis_out_stride;
  int64_t prev_start;
  int prev_len;
};

__device__ __forceinline__ void put_elem(uint8_t* row, int64_t col, int esize, uint32_t bits) {
  if (esize == 2)
    reinterpret_cast<uint16_t*>(row)[col] = (uint16_t)bits;
  else
    reinterpret_cast<uint32_t*>(row)[col] = bits;
}

__global__ __launch_bounds__(256) void tree_mask_kernel(TreeMaskArgs a) {
  const int i = blockIdx.x;
  const int tid = threadIdx.x;
  uint8_t* row = a.mask + (int64_t)i * a.mask_row_bytes;
  // the previous round's tree block becomes visible prefix: cleared before this round's block is written
  // (the two may overlap)
  if (i < a.prev_len)
    for (int j = tid; j < a.prev_len; j += 256) put_elem(row, a.prev_start + j, a.esize, 0u);
  __syncthreads();
  if (i >= a.n1) return;
  const uint8_t* vrow = a.vis + (int64_t)i * a.n1;
  uint8_t* orow = a.vis_out + (int64_t)i * a.vis_out_stride;
  for (int j = tid; j < a.n1; j += 256) {
    const uint8_t v = vrow[j] != 0;
    put_elem(row, a.past + j, a.esize, v ? 0u : a.min_bits);
    orow[j] = v;
  }
  if (tid == 0) {
    a.ids[i] = i == 0 ? a.root[0] : a.tok[i - 1];
    a.pos[i] = a.start + (i == 0 ? 0 : a.dep[i - 1]);
  }
}

}  // namespace

extern "C" int mfd_verify_inputs(const int64_t* root_tokens, const int64_t* prefix_lens, const int64_t* tokens,
                                 const int64_t* depths, const int64_t* parents, int64_t tree_stride,
                                 const int64_t* mask_offsets, int64_t* ids_out, int64_t* positions_out,
                                 uint8_t* mask_out, int bs, int W, int max_depth, int32_t* err_flag, void* stream) {
  if (bs < 0 || W < 1 || W > 4096 || max_depth < 0 || tree_stride < W)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_verify_inputs: bs=%d W=%d (1..4096) max_depth=%d tree_stride=%lld",
                         bs, W, max_depth, (long long)tree_stride);
  if (bs == 0) return MFD_OK;
  if (!root_tokens || !prefix_lens || !tokens || !depths || !parents || !mask_offsets || !ids_out || !positions_out ||
      !mask_out)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_verify_inputs: null pointer");
  if ((int64_t)bs * W > 0x7FFFFFFF) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_verify_inputs: bs * W too large");
  VerifyArgs a{root_tokens, prefix_lens, tokens, depths, parents, tree_stride, mask_offsets, ids_out, positions_out,
               mask_out, W, max_depth, err_flag};
  hipLaunchKernelGGL(verify_inputs_kernel, dim3((unsigned)(bs * W)), dim3(256), (size_t)W,
                     static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

extern "C" int mfd_tree_follow(const int64_t* posterior, const int64_t* verify_ids, const int64_t* parents,
                               int64_t parent_stride, const int64_t* window, const int64_t* prefix_lens,
                               int32_t* accept_len_out, int32_t* commit_lens_out, int64_t* bonus_out,
                               int64_t* out_tokens_out, int64_t* new_seq_lens_out, int64_t* move_src_out,
                               int64_t* move_tgt_out, int64_t* hidden_index_out, int bs, int W, int L, void* stream) {
  if (bs < 0 || W < 1 || L < 1 || L > MAXL || parent_stride < W)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_follow: bs=%d W=%d L=%d (1..%d) parent_stride=%lld", bs, W, L,
                         MAXL, (long long)parent_stride);
  if (bs == 0) return MFD_OK;
  if (!posterior || !verify_ids || !parents || !window || !prefix_lens || !accept_len_out || !commit_lens_out ||
      !bonus_out || !out_tokens_out || !new_seq_lens_out || !move_src_out || !move_tgt_out || !hidden_index_out)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_follow: null pointer");
  FollowArgs a{posterior, verify_ids, parents, parent_stride, window, prefix_lens, accept_len_out, commit_lens_out,
               bonus_out, out_tokens_out, new_seq_lens_out, move_src_out, move_tgt_out, hidden_index_out, W, L};
  hipLaunchKernelGGL(tree_follow_kernel, dim3(bs), dim3(64), 0, static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

extern "C" int mfd_kv_move(const uint64_t* buf_ptrs, int nbuf, int64_t row_stride_bytes, int nseg,
                           int64_t seg_stride_bytes, int seg_bytes, int64_t max_row, const int64_t* move_src,
                           const int64_t* move_tgt, int bs, int L, int32_t* err_flag, void* stream) {
  if (bs < 0 || nbuf < 0 || nseg < 1 || L < 1 || L > MAXL || seg_bytes < 16 || (seg_bytes % 16) != 0 ||
      (row_stride_bytes % 16) != 0 || (seg_stride_bytes % 16) != 0 || max_row < 1)
    return mfd_set_error(MFD_ERR_INVALID_ARG,
                         "mfd_kv_move: bs=%d nbuf=%d nseg=%d L=%d (1..%d) seg_bytes=%d; sizes and strides must be "
                         "multiples of 16 bytes", bs, nbuf, nseg, L, MAXL, seg_bytes);
  if (bs == 0 || nbuf == 0) return MFD_OK;
  if (!buf_ptrs || !move_src || !move_tgt) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_kv_move: null pointer");
  const int tiles = (seg_bytes + TILE - 1) / TILE;
  if ((int64_t)nseg * tiles > 65535 || nbuf > 65535)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_kv_move: too many buffers or segments");
  MoveArgs a{buf_ptrs, row_stride_bytes, nseg, seg_stride_bytes, seg_bytes, move_src, move_tgt, L, tiles, max_row,
             err_flag};
  hipLaunchKernelGGL(kv_move_kernel, dim3(bs, nbuf, nseg * tiles), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

extern "C" int mfd_tree_mask(const int64_t* root_token, int64_t start, const int64_t* tokens, const int64_t* depths,
                             const uint8_t* visibility, int n1, int64_t past, void* mask, int mask_elem_bytes,
                             uint32_t mask_min_bits, int64_t mask_row_stride, int64_t mask_cols, int mask_rows,
                             int64_t* ids_out, int64_t* positions_out, uint8_t* vis_out, int64_t vis_out_stride,
                             int64_t prev_start, int prev_len, void* stream) {
  if (n1 < 1 || past < 0 || prev_len < 0 || prev_start < 0 || (mask_elem_bytes != 2 && mask_elem_bytes != 4) ||
      mask_row_stride < mask_cols)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_mask: n1=%d past=%lld prev=(%lld, %d) elem=%d", n1,
                         (long long)past, (long long)prev_start, prev_len, mask_elem_bytes);
  // every row and column written must lie inside the caller's mask buffer and the visibility buffer
  if (past + n1 > mask_cols || prev_start + prev_len > mask_cols || n1 > mask_rows || prev_len > mask_rows ||
      vis_out_stride < n1)
    return mfd_set_error(MFD_ERR_INVALID_ARG,
                         "mfd_tree_mask: tree block (rows %d, columns %lld + %d) or previous block (%d, %lld + %d) "
                         "outside the %d x %lld mask",
                         n1, (long long)past, n1, prev_len, (long long)prev_start, prev_len, mask_rows,
                         (long long)mask_cols);
  if (!root_token || !visibility || !mask || !ids_out || !positions_out || !vis_out || (n1 > 1 && (!tokens || !depths)))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_mask: null pointer");
  TreeMaskArgs a{root_token, start, tokens, depths, visibility, n1, past, static_cast<uint8_t*>(mask),
                 mask_row_stride * mask_elem_bytes, mask_elem_bytes, mask_min_bits, ids_out, positions_out, vis_out,
                 vis_out_stride, prev_start, prev_len};
  hipLaunchKernelGGL(tree_mask_kernel, dim3((unsigned)(n1 > prev_len ? n1 : prev_len)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

extern "C" int mfd_draft_prepare(const void* bonus_tokens, const void* prefix_lens, const void* req_pool_indices,
                                 const void* req_to_token, int64_t req_to_token_stride, int index_int64_flags,
                                 int64_t mask_token_id, int64_t* block_ids_out, int64_t* positions_out,
                                 int64_t* window_out, int bs, int L, int W, void* stream) {
  if (bs < 0 || L < 0 || W < 0 || req_to_token_stride < 0 || (index_int64_flags & ~15))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_draft_prepare: bs=%d L=%d W=%d stride=%lld flags=%d", bs, L, W,
                         (long long)req_to_token_stride, index_int64_flags);
  if (bs == 0 || (L == 0 && W == 0)) return MFD_OK;
  if (!bonus_tokens || !prefix_lens || !req_pool_indices || (W > 0 && (!req_to_token || !window_out)) ||
      (L > 0 && (!block_ids_out || !positions_out)))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_draft_prepare: null pointer");
  PrepareArgs a{bonus_tokens, prefix_lens, req_pool_indices, req_to_token, req_to_token_stride, index_int64_flags,
                mask_token_id, block_ids_out, positions_out, window_out, L, W};
  hipLaunchKernelGGL(draft_prepare_kernel, dim3(bs), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

extern "C" int mfd_mode_mask(const int64_t* prefix_lens, const int64_t* mask_offsets, uint8_t* mask_out, int bs,
                             int num_modes, int block_size, void* stream) {
  if (bs < 0 || num_modes < 1 || block_size < 1 || (int64_t)num_modes * block_size > 65535)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_mask: bs=%d num_modes=%d block_size=%d (K * L <= 65535)",
                         bs, num_modes, block_size);
  if (bs == 0) return MFD_OK;
  if (!prefix_lens || !mask_offsets || !mask_out) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_mask: null pointer");
  const int KL = num_modes * block_size;
  hipLaunchKernelGGL(mode_mask_kernel, dim3(bs, KL), dim3(256), 0, static_cast<hipStream_t>(stream), prefix_lens,
                     mask_offsets, mask_out, KL, block_size);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
