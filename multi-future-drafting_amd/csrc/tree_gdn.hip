// Tree gated-delta-rule verification for gfx950.
//
// Math (inference/hf/tree_gdn_kernel.py:3-6, inference/hf/qwen35_tree.py:9-20). For the nodes of one tree
// in topological order, with A_ij = beta_i e^{G_i-G_j} k_i.k_j on strict ancestors and
// P_ij = e^{G_i-G_j} q_i.k_j on ancestors-or-self:
//   u = (I + A)^{-1} R,  R_i = beta_i (v_i - e^{G_i} S0^T k_i)
//   o = E + P u,         E_i = e^{G_i} S0^T q_i
// Instead of block inverses over dense n x n blocks, the kernel uses the tree structure: the non-zeros
// of row i of T = (I + A)^{-1} sit on i's root path (at most MAXD entries), and each row follows from a
// path-local back substitution T_i[s] = -sum_{m>s} T_i[m] A_{path(i,m), path(i,s)}. With W = P T (also
// path-supported), u = T R and o = E + W R.
//
// Work split: one workgroup per (request, value head) for trees of up to 128 nodes (larger trees:
// tree_gdn_large.hip), 8 waves, wave w owning 16 of the 128 value columns; the tree part (root paths, Gram
// entries, T, W) is computed once per head, by one group of four waves while the other group runs its S0
// products; the two groups hand over through LDS counters with bounded waits (a wait that runs out flags
// MFD_DEVERR_INTERNAL and NaN-fills that workgroup's outputs instead of hanging). Global memory is read and written through buffer resources
// (wave-uniform base and range, per-lane 32-bit offsets: rows past a request's end read as zero and stores to
// them are dropped).
//   phase 0  waves 0-3: the tree context (or the walk of the parents) and the K, Q rows straight into LDS
//            (XOR-swizzled 16-byte chunks); waves 4-7: gates, then the v rows into LDS, then their S0 columns
//            into registers (in flight through the tree phases)
//   phase 1a waves 0-3: Gram entries k_i.k_j, q_i.k_j of the lower 32 x 32 blocks (MFMA), kept for ancestor
//            pairs; then their own S0 columns
//   phase 1b all waves, per 16-row tile: K S0 and Q S0 with S0 rounded to bf16 (16x16x32 MFMA) -> R
//            (bf16 hi / lo) and E, kept in registers
//   phase 2  waves 4-7 (after their 1b and the Gram entries): path coefficients a, p (two threads per node)
//   phase 3  waves 4-7: rows of T and W from one right-looking pass over the root path each (W solves the
//            same path system with p as right-hand side; one thread per node and matrix)
//   phase 5  dense T and W rows, split into bf16 hi + lo, staged in LDS over the K / Q / v rows
//   phase 6  per 16-row tile: u = T R and o = E + W R (3 MFMA per product) and the stores.
// A request whose tree is rejected (too deep, not topological, context mismatch) gets NaN outputs.
// The fp32 operands of u = T R and W R are split into bf16 pairs (hi + lo, about 2^-17 relative), so u and o
// keep fp32 accuracy in those products; S0 enters K S0 and Q S0 as bf16, as in the reference.
// The R accumulators are used as MFMA operands without data movement: the k order of a 32-node chunk is
// the C-register row order of its two 16-row tiles. E, u and o are computed transposed (value columns as
// the M index), so that each lane holds 4 consecutive columns of one node and stores 16 bytes.
#include <mutex>

#include "gdn_common.h"

namespace {
using namespace gdn;

constexpr int CROW = MAXD + 4;       // padded coefficient row (80 B: 16-byte reads of consecutive rows hit distinct banks)
constexpr int NWAVES = 8;
constexpr int NTHREADS = NWAVES * 64;
constexpr int WCOLS = D / NWAVES;    // 16 value columns per wave

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// Staged dense rows of 16-row block t: 4 arrays (T hi, T lo, W hi, W lo) x 16 rows x stage_row(t)
// elements, covering nodes [0, 32 (t / 2 + 1)) plus 8 elements of padding (the row stride in 16-byte units
// is odd, so the 16 rows of a fragment read hit distinct banks). Within each 32-node chunk, node j sits at
// position 8 ((j % 16) / 4) + 4 ((j / 16) % 2) + j % 4: the 8 nodes of one MFMA fragment are contiguous.
__host__ __device__ constexpr int stage_row(int t) { return 32 * (t / 2 + 1) + 8; }
__host__ __device__ constexpr int stage_off(int t) {
  // 64 x sum_{t' < t} stage_row(t')
  return 64 * (8 * t + 32 * ((t & 1) ? ((t >> 1) + 1) * ((t >> 1) + 1) : (t >> 1) * ((t >> 1) + 1)));
}
__device__ __forceinline__ int stage_pos(int j) { return (j & ~31) + (((j & 15) >> 2) << 3) + (((j >> 4) & 1) << 2) + (j & 3); }

// Tree context of one request: root paths, depths and ancestor masks of its nodes, computed once per tree
// (tree_ctx_kernel, or in-kernel from the parents) and shared by every layer and head. The same layout sits
// in global memory (one block per request) and in LDS, so the GDN kernel loads it with plain 16-byte copies.
template <int NMAX>
struct alignas(16) TreeMeta {
  uint32_t anc[NMAX / 32][NMAX];         // anc[w][i] bit b: node 32 w + b is an ancestor of i or i itself
  uint8_t path[NMAX][MAXD];              // path[i][s] = ancestor of i at depth s + 1 (path[i][depth-1] = i)
  int32_t depth[NMAX];                   // nodes on the root path of i (0 for i >= n)
  int32_t bad;                           // MFD_DEVERR_* bits of the tree
  int32_t n;                             // nodes of the request
  int32_t nmax;                          // NMAX of the layout
  int32_t pad;
};
static_assert(sizeof(TreeMeta<128>) % 16 == 0, "tree context blocks are copied in 16-byte chunks");

template <int NT>
struct alignas(16) GdnSmem {
  static constexpr int NMAX = 32 * NT;
  union {
    struct {
      uint16_t k[NMAX * D];              // K rows, chunk c of row r at chunk position r * 16 + (c ^ (r & 15))
      uint16_t q[NMAX * D];              // Q rows, same layout
      uint16_t v[NMAX * D];              // v rows, chunk c of row r at chunk position r * 16 + (c ^ (2 (r & 7)))
      float coefA[NMAX][CROW];           // k_i.k_j -> a_ij (slots [0, MAXD))
      float coefP[NMAX][CROW];           // q_i.k_j -> p_ij
    } kq;                                // phases 0 - 1b
    uint16_t stage[stage_off(2 * NT)];   // phases 5 - 6
  };
  float coefT[NMAX][CROW];               // T_i[s] (0 past the depth); padded rows: one row per lane is written
  float coefW[NMAX][CROW];               // W_i[s] (0 past the depth)   without bank conflicts
  TreeMeta<NMAX> meta;
  int par[NMAX];
  float G[NMAX], beta[NMAX], eG[NMAX];
  int sync[4];                           // hand-over counters of the two wave groups
};

struct GdnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* g_cum;
  const float* beta;
  const float* s0;
  const int32_t* parents;
  const int8_t* anc8;
  const int32_t* cu_nodes;
  const uint8_t* ctx;  // tree contexts (TreeMeta blocks, one per request) or NULL
  float* u;
  float* o;
  int32_t* err;
  int R, N, HK, H;
  int csplit;  // value-column blocks per (request, value head): 1, 2 or 4 (small grids; the kernel's CS)
};


enum { SYNC_GRAM = 0, SYNC_V = 1, SYNC_COEF = 2 };

// Hand-over between the wave groups of a workgroup through an LDS counter: each wave of a group signals once
// after its LDS writes (and, for direct-to-LDS data, after its own vmcnt wait) have completed; a waiting wave
// polls the counter. LDS is coherent within the workgroup, so a completed write is seen by the next read.
__device__ __forceinline__ void group_signal(int* c) {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
  if ((threadIdx.x & 63) == 0) atomicAdd(c, 1);
}
// Wait until the counter reaches target; false if it did not within a bound far above any real wait
// (2^20 polls with a short sleep between them: tens of milliseconds).
__device__ __forceinline__ bool group_wait(const int* c, int target) {
  for (int it = 0; it < (1 << 20); ++it) {
    const int v = __builtin_amdgcn_readfirstlane(__atomic_load_n(c, __ATOMIC_RELAXED));
    if (v >= target) {
      asm volatile("" ::: "memory");
      return true;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

__device__ __forceinline__ bf16x8 ld_lds8(const uint16_t* p) { return as_bf16x8(*reinterpret_cast<const u16x8*>(p)); }

// Root path, depth and ancestor mask of node i < NMAX from the parent pointers in LDS: one walk up the
// parents, the chain kept in registers. Nodes i >= n get depth 0 and an empty mask. Sets MFD_DEVERR_* bits
// in m.bad for a parent that does not precede its child and for a root path longer than MAXD nodes.
template <int NMAX>
__device__ __forceinline__ void walk_root_path(TreeMeta<NMAX>& m, const int* par, int i, int n) {
  int d = 0;
  uint32_t msk[NMAX / 32];
#pragma unroll
  for (int x = 0; x < NMAX / 32; ++x) msk[x] = 0u;
  if (i < n) {
    int chain[MAXD + 1];
    int cur = i;
#pragma unroll
    for (int s = 0; s <= MAXD; ++s) {
      chain[s] = cur;
      if (cur >= 0) {
#pragma unroll
        for (int x = 0; x < NMAX / 32; ++x)
          if ((cur >> 5) == x) msk[x] |= 1u << (cur & 31);
        const int p = par[cur];
        if (p >= cur || p < -1) {
          atomicOr(&m.bad, MFD_DEVERR_NOT_TOPOLOGICAL);
          cur = -1;
        } else {
          cur = p;
        }
        ++d;
      }
    }
    if (cur >= 0 || d > MAXD) {
      atomicOr(&m.bad, MFD_DEVERR_TOO_DEEP);
    } else {
#pragma unroll
      for (int s = 0; s < MAXD; ++s)
        if (s < d) m.path[i][d - 1 - s] = (uint8_t)chain[s];
    }
  }
  m.depth[i] = d;
#pragma unroll
  for (int x = 0; x < NMAX / 32; ++x) m.anc[x][i] = msk[x];
}

template <int NT, bool CTX, int CS>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void tree_gdn_kernel(GdnArgs a) {
  using S = GdnSmem<NT>;
  constexpr int NMAX = S::NMAX;
  constexpr int NT16 = 2 * NT;
  __shared__ S sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4;    // 16x16 tiles: lane group
  const int l16 = lane & 15;

  // ---- workgroup -> (request, key head, GQA member, value-column block); the members of one (request, key
  //      head) share the q / k rows and land on the same XCD (workgroup id modulo 8). With CS > 1 (grids too
  //      small to fill the chip) each workgroup computes the tree part of its head in full but only D / CS
  //      value columns, on waves 0 .. 8 / CS - 1.
  const int G = a.H / a.HK;
  const int P = a.R * a.HK;
  const int P8 = (P + 7) >> 3;
  const int id = blockIdx.x;
  const int rest = id >> 3;
  const int pidx = (rest % P8) * 8 + (id & 7);
  if (pidx >= P) return;
  const int mem = (rest / P8) % G;
  const int cblk = rest / (P8 * G);
  constexpr int ccols = D / CS;                      // value columns of this workgroup
  const bool own = CS == 1 || w < NWAVES / CS;       // this wave owns 16 of them
  const int col0 = cblk * ccols + (own ? w : 0) * WCOLS;  // its first value column
  const int r = pidx / a.HK;
  const int hk = pidx % a.HK;
  const int h = hk * G + mem;

  int ns_, n_;
  request_range(a.cu_nodes, r, a.N, ns_, n_);
  const int ns = __builtin_amdgcn_readfirstlane(ns_);
  const int n = __builtin_amdgcn_readfirstlane(n_);
  if (n <= 0) return;
  if (n > NMAX) {
    nan_fill(a.u, a.o, ns, n, a.H, h, cblk * ccols, ccols, tid, NTHREADS);
    if (tid == 0 && a.err) atomicOr(a.err, MFD_DEVERR_TOO_MANY_NODES);
    return;
  }
  const int nt16 = (n + 15) >> 4;
  const size_t rh = (size_t)r * a.H + h;
  const int HD = a.H * D, HKD = a.HK * D;  // node strides of v / u / o and of q / k (elements)

  // buffer resources of this workgroup's slices (ranges in bytes: rows past n read as zero)
  const __amdgpu_buffer_rsrc_t rs_s0 = rsrc(a.s0 + rh * D * D, D * D * 4);
  const __amdgpu_buffer_rsrc_t rs_u = rsrc(a.u + ((size_t)ns * a.H + h) * D, (uint32_t)n * HD * 4);
  const __amdgpu_buffer_rsrc_t rs_o = rsrc(a.o + ((size_t)ns * a.H + h) * D, (uint32_t)n * HD * 4);
  const uint16_t* kbase = a.k + ((size_t)ns * a.HK + hk) * D;
  const uint16_t* qbase = a.q + ((size_t)ns * a.HK + hk) * D;

  // ---- phase 0: waves 0-3 issue the tree context (when given) and the K / Q rows, direct-to-LDS; waves 4-7
  //      load the gates (and the parents), then issue the v rows (direct-to-LDS) and, without a tree
  //      context, walk the root paths while the K / Q rows are in flight. The split keeps the node loads
  //      out of the DMA waves, whose vector memory counter retires in order.
  constexpr int NKQ = NMAX / 16;  // K (and Q) direct loads per DMA wave: 4 rows each
  constexpr int NV = NMAX / 16;   // v direct loads per node wave
  constexpr int NCM = (int)(sizeof(TreeMeta<NMAX>) / 16);  // 16-byte chunks of a tree context
  const int nw = tid - 256;       // node index of the threads of waves 4-7
  if (w < 4) {
    if constexpr (CTX) {
      const uint8_t* cbase = a.ctx + (size_t)r * sizeof(TreeMeta<NMAX>);
      const uint32_t lds_m = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) TreeMeta<NMAX>*)&sm.meta;
#pragma unroll
      for (int x = 0; x < (NCM + 255) / 256; ++x) {
        const int c = x * 256 + w * 64 + lane;
        if (c < NCM) dma16_s(cbase, (uint32_t)c * 16u, lds_m + (uint32_t)((x * 256 + w * 64) * 16));
      }
    }
    const uint32_t lds_k = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)sm.kq.k;
    const uint32_t lds_q = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)sm.kq.q;
    // instruction x fills chunk positions (w NKQ + x) 64 + lane: row (w NKQ + x) 4 + lane / 16; rows
    // past n read row n - 1 (never used: their masks and R rows are zero)
#pragma unroll
    for (int x = 0; x < NKQ; ++x) {
      const int row = (w * NKQ + x) * 4 + (lane >> 4);
      const int c = (lane & 15) ^ (row & 15);
      const int rc = row < n ? row : n - 1;
      const uint32_t off = (uint32_t)(rc * HKD + c * 8) * 2u;
      dma16_s(kbase, off, lds_k + (uint32_t)((w * NKQ + x) * 1024));
      dma16_s(qbase, off, lds_q + (uint32_t)((w * NKQ + x) * 1024));
    }
  } else if (nw < NMAX) {
    float g_own = 0.f, b_own = 0.f;
    if (nw < n) {
      g_own = a.g_cum[(size_t)(ns + nw) * a.H + h];
      b_own = a.beta[(size_t)(ns + nw) * a.H + h];
    }
    if constexpr (!CTX) sm.par[nw] = (nw < n) ? parent_of(a.parents, a.anc8, ns, nw, n) : -1;
    sm.G[nw] = g_own;
    sm.eG[nw] = __expf(g_own);
    sm.beta[nw] = b_own;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < MAXD; s += 4) {
      *reinterpret_cast<f32x4*>(&sm.kq.coefA[nw][s]) = z;
      *reinterpret_cast<f32x4*>(&sm.kq.coefP[nw][s]) = z;
    }
  }
  if constexpr (!CTX) {
    if (tid == 0) sm.meta.bad = 0;
  }
  if (tid < 4) sm.sync[tid] = 0;
  __syncthreads();
  if (w >= 4) {
    const uint32_t lds_v = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)sm.kq.v;
    const uint16_t* vbase = a.v + ((size_t)ns * a.H + h) * D;
#pragma unroll
    for (int x = 0; x < NV; ++x) {
      const int row = ((w - 4) * NV + x) * 4 + (lane >> 4);
      const int c = (lane & 15) ^ ((row & 7) << 1);
      const int rc = row < n ? row : n - 1;
      dma16_s(vbase, (uint32_t)(rc * HD + c * 8) * 2u, lds_v + (uint32_t)(((w - 4) * NV + x) * 1024));
    }
    if constexpr (!CTX) {
      if (nw < NMAX) walk_root_path(sm.meta, sm.par, nw, n);
    }
  }
  if (w < 4) wait_vmcnt<0>();  // tree context and K / Q rows (direct-to-LDS loads are not tracked by the compiler)
  __syncthreads();
  if constexpr (CTX) {
    // a context built for another request size or another max_nodes
    if (tid == 0 && (sm.meta.n != n || sm.meta.nmax != NMAX)) sm.meta.bad |= MFD_DEVERR_BAD_CONTEXT;
    __syncthreads();
  }
  if (sm.meta.bad) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no load of this workgroup may outlive it
    nan_fill(a.u, a.o, ns, n, a.H, h, cblk * ccols, ccols, tid, NTHREADS);
    if (tid == 0 && a.err) atomicOr(a.err, sm.meta.bad);
    return;
  }
  // this lane's S0 column (B fragments of 16x16x32, k = 32c + 8 g4 + e), consumed in phase 1b, in flight
  // through the tree phases. Issued once the K / Q rows have landed (so that the K / Q requests of all
  // workgroups reach memory first): before the Gram blocks for trees of at most 64 nodes, after them for
  // larger trees, whose Gram phase is long enough for the v requests to drain from the memory queues first
  // (issued before it, these loads hold the waves up behind the v requests).
  // S0 is row-major ([d_k][d_v]) and a fragment wants 8 rows of one column, so the loads are 16-byte row pieces
  // transposed within each quad of lanes: lane 4q + i of a 16-lane group loads row 32c + 8 g4 + 4h + i,
  // columns 16w + 4q .. + 3 (one load per (c, h): 8 per lane instead of 32 single floats), and two rounds of
  // quad exchanges (lanes i ^ 1, then i ^ 2) leave lane 4q + i with column 16w + 4q + i of the quad's 4 rows.
  u32x4 s0v[D / 32][2];
  constexpr int NS0 = (D / 32) * 2;  // S0 loads per lane (vector memory operations of issue_s0)
  auto issue_s0 = [&]() __attribute__((always_inline)) {
    const uint32_t voff = (uint32_t)((g4 * 8 + (l16 & 3)) * D + col0 + (l16 & ~3)) * 4u;
#pragma unroll
    for (int c = 0; c < D / 32; ++c)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        s0v[c][hh] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_s0, voff, (c * 32 + 4 * hh) * D * 4, 2));
  };
  // fragment of row 16 blk + l16, k = 32 c + 8 g4 + e: chunk 4c + g4 of the row, swizzled by l16
  auto frag = [&](const uint16_t* rows, int blk, int c) __attribute__((always_inline)) {
    return ld_lds8(&rows[(blk * 16 + l16) * D + (((4 * c + g4) ^ l16) << 3)]);
  };

  // Two wave groups run side by side from here to the last barrier, handing data over through LDS counters
  // instead of workgroup barriers (so that one group's VALU work overlaps the other's MFMA work):
  //   waves 0-3: Gram blocks (phase 1a) -> signal -> their S0 column -> phase 1b
  //   waves 4-7: their S0 column (requested right away) -> phase 1b -> wait for the Gram -> phase 2 -> phase 3
  // Every wait is bounded: a wait that runs out (it never should) goes on, so the workgroup always completes, and
  // at the next barrier the workgroup's outputs become NaN and MFD_DEVERR_INTERNAL is set.
  bool stuck = false;
  // S0 columns: waves 4-7 request theirs right away; with CS > 1 the owning waves (all in 0-3) do too,
  // since the small grid leaves the memory system idle
  if (own && (w >= 4 || CS > 1)) issue_s0();
  if (w < 4) {
    // ---- phase 1a: Gram blocks (T, J), J <= T, of 32 x 32 nodes (32x32x16 MFMA: each fragment read feeds
    //      twice the work of a 16x16 block, and the phase is bound by LDS reads), numbered row by row; wave w
    //      takes blocks w, w + 4, ...
    const int g2 = lane >> 5;
    const int l32 = lane & 31;
    const int nt32 = (n + 31) >> 5;
    const int nb = nt32 * (nt32 + 1) / 2;
    // fragment of row 32 blk + l32, dims 16 ks + 8 g2 .. + 7: chunk 2 ks + g2 of the row, swizzled by the row
    auto frag32 = [&](const uint16_t* rows, int blk, int ks) __attribute__((always_inline)) {
      const int r = blk * 32 + l32;
      return ld_lds8(&rows[r * D + (((2 * ks + g2) ^ (r & 15)) << 3)]);
    };
    for (int b = w; b < nb; b += 4) {
      int T = 0, J = b;
      while (J > T) {
        J -= T + 1;
        ++T;
      }
      f32x16 gkk = {}, gqk = {};
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const bf16x8 bk = frag32(sm.kq.k, J, ks);
        gkk = mfma32(frag32(sm.kq.k, T, ks), bk, gkk);
        gqk = mfma32(frag32(sm.kq.q, T, ks), bk, gqk);
      }
      // C register r: row i = 32 T + 8 (r / 4) + 4 g2 + r % 4, column j = 32 J + l32. j is an ancestor-or-self
      // of i iff bit j of i's mask is set; its slot on i's path is depth(j) - 1.
      const int j = J * 32 + l32;
      const int sj = sm.meta.depth[j] - 1;
      const uint32_t bit = 1u << l32;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i0 = T * 32 + 8 * q + 4 * g2;
        const u32x4 mw = *reinterpret_cast<const u32x4*>(&sm.meta.anc[J][i0]);
        // 24-bit multiply for the LDS offset: a 32-bit multiply-add is emitted as v_mad_u64_u32, whose
        // undefined high addend register can alias a load still in flight and force a wait for it
        const int o0 = (int)__umul24((unsigned)i0, (unsigned)CROW) + sj;
        // only ancestor pairs are written (lanes of other pairs are masked off: writing them to a per-lane
        // sink slot instead cost LDS bank conflicts with the row writes)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool anc = (mw[e] & bit) != 0;
          if (anc) {
            (&sm.kq.coefP[0][0])[o0 + e * CROW] = gqk[4 * q + e];
            if (j < i0 + e) (&sm.kq.coefA[0][0])[o0 + e * CROW] = gkk[4 * q + e];
          }
        }
      }
    }
    group_signal(&sm.sync[SYNC_GRAM]);
    if (CS == 1) issue_s0();
  } else {
    // this wave's v rows have landed: only its NS0 S0 loads (when it owns value columns) are younger
    if (own)
      wait_vmcnt<NS0>();
    else
      wait_vmcnt<0>();
    group_signal(&sm.sync[SYNC_V]);
  }
  stuck |= !group_wait(&sm.sync[SYNC_V], 4);  // both groups' phase 1b reads every v row

  // R as bf16 pairs: [32-node chunk][hi, lo] dword x: rows 32c + 16 (x / 2) + 4 g4 + 2 (x % 2) + {0, 1}
  // (element e < 4: row 32c + 4 g4 + e, e >= 4: row 32c + 16 + 4 g4 + e - 4), C layout: lane = value
  // column. E^T: lane = node 16 t + l16, value columns 4 g4 + rr. (Waves that own no value columns skip 1b.)
  u32x4 Rb[NT][2];
  f32x4 oacc[NT16];
  if (own) {
  // S0 enters K S0 and Q S0 rounded to bf16 (nearest even), as in the reference (s_blk,
  // inference/hf/tree_gdn_kernel.py:107); the products accumulate in fp32
  bf16x8 sh[D / 32];
  {
    const bool odd = (lane & 1) != 0, hi2 = (lane & 2) != 0;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      u32x4 hv;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u32x4 x = s0v[c][hh];  // row 4 hh + i of this chunk, columns 4q .. 4q + 3
        // round 1 (lanes i ^ 1): z[j] = x[j] if j % 2 == i % 2, else the partner's x[j ^ 1]
        u32x4 z;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const uint32_t send = odd ? x[2 * p] : x[2 * p + 1];
          const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xB1, 0xF, 0xF, false);  // quad [1,0,3,2]
          z[2 * p] = odd ? got : x[2 * p];
          z[2 * p + 1] = odd ? x[2 * p + 1] : got;
        }
        // round 2 (lanes i ^ 2): y[j] = z[j] if j / 2 == i / 2, else the partner's z[j ^ 2]
        u32x4 y;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const uint32_t send = hi2 ? z[p] : z[p + 2];
          const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0x4E, 0xF, 0xF, false);  // quad [2,3,0,1]
          y[p] = hi2 ? got : z[p];
          y[p + 2] = hi2 ? z[p + 2] : got;
        }
        // y[j]: row 32c + 8 g4 + 4 hh + j of this lane's column
#pragma unroll
        for (int e = 0; e < 2; ++e)
          hv[2 * hh + e] = __builtin_bit_cast(
              uint32_t, __builtin_convertvector((f32x2){__uint_as_float(y[2 * e]), __uint_as_float(y[2 * e + 1])}, bf16x2));
      }
      sh[c] = __builtin_bit_cast(bf16x8, hv);
    }
  }
  // v entries of the R rows by the LDS transpose read: lane 4e + q of a 16-lane group addresses row
  // 16 t + 4 g4 + e, columns 16 w + 4 q .. + 3, and lane j receives column 16 w + j of the 4 rows
  const uint16_t* vrow = &sm.kq.v[(g4 * 4 + (l16 >> 2)) * D];
  const int vchunk = (col0 >> 3) + ((l16 & 3) >> 1);
  const int vhalf = (l16 & 1) * 4;
  bf16x8 fk[2][D / 32], fq[2][D / 32];
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    fk[0][c] = frag(sm.kq.k, 0, c);
    fq[0][c] = frag(sm.kq.q, 0, c);
  }
#pragma unroll
  for (int t = 0; t < NT16; ++t) {
    const int bsel = t & 1;
    if (t + 1 < nt16) {
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        fk[bsel ^ 1][c] = frag(sm.kq.k, t + 1, c);
        fq[bsel ^ 1][c] = frag(sm.kq.q, t + 1, c);
      }
    }
    f32x4 ak = {0.f, 0.f, 0.f, 0.f}, eq = ak;
    if (t < nt16) {
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        ak = mfma16(fk[bsel][c], sh[c], ak);
        eq = mfma16(sh[c], fq[bsel][c], eq);
      }
    }
    const int i0 = t * 16 + g4 * 4;
    const int rv0 = t * 16 + g4 * 4 + (l16 >> 2);  // row this lane addresses in the transpose read
    const v4i16 vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16*)&vrow[t * 16 * D + ((vchunk ^ ((rv0 & 7) << 1)) << 3) + vhalf]);
    const bf16x4 vv = __builtin_bit_cast(bf16x4, vt);
    const f32x4 bi = *reinterpret_cast<const f32x4*>(&sm.beta[i0]);
    const f32x4 ei = *reinterpret_cast<const f32x4*>(&sm.eG[i0]);
    float rv[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) rv[rr] = (i0 + rr < n) ? bi[rr] * ((float)vv[rr] - ei[rr] * ak[rr]) : 0.f;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      uint32_t h2, l2;
      split2_bf16(rv[2 * x], rv[2 * x + 1], h2, l2);
      Rb[t >> 1][0][(t & 1) * 2 + x] = h2;
      Rb[t >> 1][1][(t & 1) * 2 + x] = l2;
    }
    const int il = t * 16 + l16;
    const float el = (il < n) ? sm.eG[il] : 0.f;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) oacc[t][rr] = el * eq[rr];
  }
  }  // own
  if (w >= 4) {
    const int t2 = tid - 256;  // thread index within the group
    stuck |= !group_wait(&sm.sync[SYNC_GRAM], 4);
    // ---- phase 2 (two threads per node; thread h of node i owns the path slots 8 h .. 8 h + 7):
    //      a_ij = beta_i e^{G_i-G_j} k_i.k_j (strict), p_ij = e^{G_i-G_j} q_i.k_j
    {
      const int qn = t2 >> 1;
      const int qh = t2 & 1;
      if (qn < n) {
        const float gi = sm.G[qn];
        const float bi = sm.beta[qn];
        const int qdep = sm.meta.depth[qn];
        const u32x2 pq = *reinterpret_cast<const u32x2*>(&sm.meta.path[qn][8 * qh]);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int s0i = 8 * qh + 4 * hh;
          f32x4 xa = *reinterpret_cast<const f32x4*>(&sm.kq.coefA[qn][s0i]);
          f32x4 xp = *reinterpret_cast<const f32x4*>(&sm.kq.coefP[qn][s0i]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int s = s0i + e;
            const int j = (s < qdep) ? (int)((pq[hh] >> (8 * e)) & 0xFFu) : qn;
            const float ex = __expf(gi - sm.G[j]);
            xp[e] = (s < qdep) ? xp[e] * ex : 0.f;
            xa[e] = (s < qdep - 1) ? xa[e] * (bi * ex) : 0.f;
          }
          *reinterpret_cast<f32x4*>(&sm.kq.coefA[qn][s0i]) = xa;
          *reinterpret_cast<f32x4*>(&sm.kq.coefP[qn][s0i]) = xp;
        }
      }
    }
    group_signal(&sm.sync[SYNC_COEF]);
    stuck |= !group_wait(&sm.sync[SYNC_COEF], 4);
    // ---- phase 3 (one thread per node and matrix): rows of T = (I + A)^{-1} and of W = P T from one right-looking pass
    //      over the root path. Row i of T solves x L = e_{d-1} and row i of W solves x L = p_i, with L = I + A
    //      restricted to the path (unit lower triangular, L[m][s] = a_{path(m)}[s]), so both take
    //      x[m] = rhs[m] - sum_{k>m} x[k] a_{path(k)}[m] and share the a-row reads.
    // T rows on threads t2 < NMAX, W rows on threads NMAX .. 2 NMAX - 1 (whole waves each): the two solves share
    // the a-row reads but are independent, so each thread runs one chain of FMAs
    const int which = t2 >= NMAX ? 1 : 0;
    const int i = t2 - which * NMAX;
    if (t2 < 2 * NMAX && i < n) {
      const int dep = sm.meta.depth[i];
      int pth[MAXD];
      float rhs[MAXD], acc[MAXD], X[MAXD];
#pragma unroll
      for (int s4 = 0; s4 < MAXD; s4 += 4) {
        const uint32_t pw = *reinterpret_cast<const uint32_t*>(&sm.meta.path[i][s4]);
        const f32x4 xp = *reinterpret_cast<const f32x4*>(&sm.kq.coefP[i][s4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pth[s4 + e] = (s4 + e < dep) ? (int)((pw >> (8 * e)) & 0xFFu) : i;
          // T: x L = e_{d-1}; W: x L = p_i
          rhs[s4 + e] = which ? xp[e] : ((s4 + e == dep - 1) ? 1.f : 0.f);
          acc[s4 + e] = 0.f;
        }
      }
#pragma unroll
      for (int m = MAXD - 1; m >= 0; --m) {
        const bool on = m < dep;
        const float xm = on ? rhs[m] - acc[m] : 0.f;
        X[m] = xm;
        if (m > 0) {
          const int j = pth[m];
#pragma unroll
          for (int s4 = 0; s4 < m; s4 += 4) {
            const f32x4 row = *reinterpret_cast<const f32x4*>(&sm.kq.coefA[j][s4]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (s4 + e < m) acc[s4 + e] = fmaf(xm, row[e], acc[s4 + e]);
          }
        }
      }
      float* dst = which ? &sm.coefW[i][0] : &sm.coefT[i][0];
#pragma unroll
      for (int s = 0; s < MAXD; s += 4) *reinterpret_cast<f32x4*>(dst + s) = (f32x4){X[s], X[s + 1], X[s + 2], X[s + 3]};
    }
  }
  // the K / Q / v rows and the a / p coefficients are dead; T and W rows are complete. A hand-over wait that ran
  // out leaves the LDS rows unreliable: this workgroup's outputs become NaN instead (never silent)
  if (__syncthreads_or(stuck ? 1 : 0)) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no load of this workgroup may outlive it
    nan_fill(a.u, a.o, ns, n, a.H, h, cblk * ccols, ccols, tid, NTHREADS);
    if (tid == 0 && a.err) atomicOr(a.err, MFD_DEVERR_INTERNAL);
    return;
  }

  // ---- phase 5: dense T and W rows of every block: zero fill by all threads, then the path entries
  {
    constexpr int NCH = stage_off(NT16) / 8;  // 16-byte chunks
    const u16x8 zz = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int x = 0; x < (NCH + NTHREADS - 1) / NTHREADS; ++x)
      if (x * NTHREADS + tid < NCH) *reinterpret_cast<u16x8*>(&sm.stage[8 * (x * NTHREADS + tid)]) = zz;
  }
  __syncthreads();
#pragma unroll
  for (int x = 0; x < NMAX * MAXD / NTHREADS + (NMAX * MAXD % NTHREADS != 0); ++x) {
    const int idx = x * NTHREADS + tid;
    const int i = idx >> 4;  // MAXD = 16 slots per row
    const int s = idx & 15;
    const int ic = i < NMAX ? i : NMAX - 1;
    const int di = sm.meta.depth[ic];
    const int j = sm.meta.path[ic][s];
    const float tv = sm.coefT[ic][s];
    const float wv = sm.coefW[ic][s];
    const int t = ic >> 4;
    const int rs = stage_row(t);
    // only path slots of rows below n are written (the other lanes are masked off)
    const bool on = i < n && s < di;
    if (on) {
      uint16_t* const p0 = &sm.stage[stage_off(t) + (i & 15) * rs + stage_pos(j)];
      const int step = 16 * rs;
      __bf16 hi, lo;
      split_bf16(tv, hi, lo);
      p0[0] = __builtin_bit_cast(uint16_t, hi);
      p0[step] = __builtin_bit_cast(uint16_t, lo);
      split_bf16(wv, hi, lo);
      p0[2 * step] = __builtin_bit_cast(uint16_t, hi);
      p0[3 * step] = __builtin_bit_cast(uint16_t, lo);
    }
  }
  __syncthreads();

  // ---- phase 6: per 16-row tile t: u^T = R^T T^T, o^T = E^T + R^T W^T (lane = node 16 t + l16, value
  //      columns 4 g4 + rr), 16-byte stores
  if (!own) return;
  const uint32_t st_off = (uint32_t)(l16 * HD + col0 + g4 * 4) * 4u;
#pragma unroll
  for (int t = 0; t < NT16; ++t) {
    if (t >= nt16) break;
    f32x4 uacc = {0.f, 0.f, 0.f, 0.f}, oa = oacc[t];
    f32x4 uc1 = uacc, uc2 = uacc, oc1 = uacc, oc2 = uacc;  // the hi x lo and lo x hi terms, summed at the end
    const uint16_t* st = &sm.stage[stage_off(t) + l16 * stage_row(t) + g4 * 8];
#pragma unroll
    for (int kc = 0; kc <= (t >> 1); ++kc) {
      const int rsz = stage_row(t);
      const bf16x8 thi = ld_lds8(st + kc * 32);
      const bf16x8 tlo = ld_lds8(st + 16 * rsz + kc * 32);
      const bf16x8 whi = ld_lds8(st + 32 * rsz + kc * 32);
      const bf16x8 wlo = ld_lds8(st + 48 * rsz + kc * 32);
      const bf16x8 rhi = __builtin_bit_cast(bf16x8, Rb[kc][0]);
      const bf16x8 rlo = __builtin_bit_cast(bf16x8, Rb[kc][1]);
      uacc = mfma16(rhi, thi, uacc);
      oa = mfma16(rhi, whi, oa);
      uc1 = mfma16(rlo, thi, uc1);
      oc1 = mfma16(rlo, whi, oc1);
      uc2 = mfma16(rhi, tlo, uc2);
      oc2 = mfma16(rhi, wlo, oc2);
    }
    uacc += uc1 + uc2;
    oa += oc1 + oc2;
    // rows past n fall outside the buffer ranges: those stores are dropped. Store data goes through VGPRs one
    // element at a time (the empty asm): built straight from the accumulator registers, the stored vector held
    // element 0 four times in this compiler's output. The whole offset goes into the VGPR offset (soffset stays
    // the constant 0): the compiler's guard against a VALU write to a 16-byte store's data registers right
    // after the store issues (which loses store data) is not applied to stores whose soffset is an SGPR.
    u32x4 uv, ov;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      float x = uacc[rr], y = oa[rr];
      asm volatile("" : "+v"(x), "+v"(y));
      uv[rr] = __builtin_bit_cast(uint32_t, x);
      ov[rr] = __builtin_bit_cast(uint32_t, y);
    }
    __builtin_amdgcn_raw_buffer_store_b128(uv, rs_u, st_off + (uint32_t)(t * 16 * HD * 4), 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(ov, rs_o, st_off + (uint32_t)(t * 16 * HD * 4), 0, 0);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// tree_gdn_pipe_kernel: one workgroup per (request, value head) for grids that fill the chip, trees of up to
// 32 NT nodes. Two groups of four waves, handing data over through LDS counters (bounded waits):
//   tree waves (0-3): the tree part, which needs only the K / Q rows and the gates: K / Q rows straight into MFMA
//     fragments (and into LDS for the other waves); Gram blocks of 16 x 16 nodes, kept for ancestor pairs and
//     scaled on the way into the path coefficients a and p; rows of T and W by path-local back substitution, into
//     LDS as fp16 rows scaled by a power of two
//   column waves (4-7): LDS clears; the S0 and v pieces of their 32 value columns, S0 straight into MFMA fragments
//     (transposed within quads of lanes); R = beta (v - e^G K S0) for every node of their columns, scaled per
//     column by a power of two into fp16; then, once T and W are staged, per tile E^T = e^G S0^T Q^T,
//     u^T = R^T T^T and o^T = E^T + R^T W^T (the products hide behind the stores)
// The 2 NT tiles of 16 nodes are paired (p, 2 NT - 1 - p) for the tree waves, which gives every pair the same Gram
// work (4 / NT tree waves per pair). fp16 products: the MFMA accumulates in fp32 and the power-of-two scales come
// off exactly afterwards (about 2^-11 relative per operand).
template <int NT>
struct alignas(16) PipeSmem {
  static constexpr int NMAX = 32 * NT;
  static constexpr int NT16 = 2 * NT;
  static constexpr int KROW = D + 8;  // padded K / Q row (bf16): 16-byte reads of 16 rows hit distinct banks
  // staged T / W rows of tile t: 16 rows of srow(t) fp16 (nodes [0, 32 (t / 2 + 1)) plus 8 of padding)
  static constexpr int srow(int t) { return 32 * (t / 2 + 1) + 8; }
  static constexpr int soff(int t) {
    return 16 * (8 * t + 32 * ((t & 1) ? ((t >> 1) + 1) * ((t >> 1) + 1) : (t >> 1) * ((t >> 1) + 1)));
  }
  static constexpr int STAGE = soff(NT16);
  uint16_t kr[NMAX * KROW];        // K rows: the Gram blocks' second operand and R's first
  uint16_t qr[NMAX * KROW];        // Q rows: E's second operand
  uint16_t st[2][STAGE];           // T and W rows, fp16, row-scaled
  // coefficient rows, each followed by sink words: the targets of the Gram scatter's non-ancestor entries (never
  // read). A sink lies at the same distance from its rows in both matrices, so one select of an entry's offset
  // serves the a and the p write.
  // >= 64 lanes + 3 CROW (entries e = 0 .. 3 of a lane at e CROW), a multiple of 4 (16-byte aligned rows), and with
  // the a-to-p distance not a multiple of 256 bytes: the compiler then keeps the a and p writes apart, each with the
  // entry's e CROW in its immediate offset, instead of pairing them in one write2st64 behind an address add per entry
  static constexpr int SINKW = 132;
  float coefA[NMAX][CROW];
  float sinkA[SINKW];
  float coefP[NMAX][CROW];
  float sinkP[SINKW];
  TreeMeta<NMAX> meta;
  int par[NMAX];
  float G[NMAX], beta[NMAX], eG[NMAX];  // G in units of log2 (g_cum log2(e)): e^{G_i - G_j} = exp2(G_i - G_j)
  int rexp[2][NMAX];               // row exponents of T and W
  int cexp[D];                     // column exponents of R
  int sync[8];                     // hand-over counters
};
// PS_TWT + w: tree wave w's T and W rows are staged (NT = 4: the rows of tiles 2 w and 2 w + 1)
enum { PS_CLEAR = 0, PS_TREE = 1, PS_COEF = 2, PS_TW = 3, PS_TWT = 4 };

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f32x4 mfma16_f16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Gram blocks (t, t') of tile t for the column tiles t' = tp0, tp0 + step, ... (nvalid <= GBN of them): k_i.k_j and
// q_i.k_j (A = the tile's K / Q fragments, lane: node 16 t + l16, dims 32 kc + 8 g4 .. + 7; B = K rows from LDS), kept
// for ancestor pairs as the path coefficients a_ij = beta_i e^{G_i - G_j} k_i.k_j (strict ancestors) and
// p_ij = e^{G_i - G_j} q_i.k_j (ancestors and self) at slot s = depth(j) - 1. C register e: row i = 16 t + 4 g4 + e,
// column j = 16 t' + l16. A block's masks, depths and gates are read before its products; lanes of non-ancestor
// pairs write to their own sink word (no exec-mask branches).
template <int GBN, typename S>
__device__ __forceinline__ void pipe_gram_blocks(S& sm, const u32x4 (&ka)[D / 32], const u32x4 (&qa)[D / 32], int t,
                                                 int tp0, int step, int nvalid, int lane) {
  const int g4 = lane >> 4, l16 = lane & 15;
  const int i0 = t * 16 + g4 * 4;
  int jn[GBN], sj[GBN];
  float gj[GBN];
  u32x4 mw[GBN];
  bf16x8 bb[GBN][D / 32];
#pragma unroll
  for (int q = 0; q < GBN; ++q) {
    const int tp = tp0 + (q < nvalid ? q : 0) * step;
    jn[q] = tp * 16 + l16;
    sj[q] = sm.meta.depth[jn[q]] - 1;
    gj[q] = sm.G[jn[q]];
    mw[q] = *reinterpret_cast<const u32x4*>(&sm.meta.anc[jn[q] >> 5][i0]);
    const uint16_t* br = &sm.kr[__umul24((unsigned)jn[q], (unsigned)S::KROW) + g4 * 8];
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc) bb[q][kc] = ld_lds8(br + kc * 32);
  }
  const f32x4 gi = *reinterpret_cast<const f32x4*>(&sm.G[i0]);
  const f32x4 bi = *reinterpret_cast<const f32x4*>(&sm.beta[i0]);
  f32x4 gk[GBN], gq[GBN];
#pragma unroll
  for (int q = 0; q < GBN; ++q) gk[q] = gq[q] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kc = 0; kc < D / 32; ++kc)
#pragma unroll
    for (int q = 0; q < GBN; ++q) {
      gk[q] = mfma16(__builtin_bit_cast(bf16x8, ka[kc]), bb[q][kc], gk[q]);
      gq[q] = mfma16(__builtin_bit_cast(bf16x8, qa[kc]), bb[q][kc], gq[q]);
    }
  float* const cA = &sm.coefA[0][0];
  float* const cP = &sm.coefP[0][0];
#pragma unroll
  for (int q = 0; q < GBN; ++q) {
    if (q >= nvalid) break;
    const uint32_t bit = 1u << (jn[q] & 31);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = (int)__umul24((unsigned)(i0 + e), (unsigned)CROW);
      const bool anc = (mw[q][e] & bit) != 0;
      const float dec = __builtin_amdgcn_exp2f(gi[e] - gj[q]);
      *(anc ? cP + row + sj[q] : sm.sinkP + lane) = gq[q][e] * dec;
      *((anc && jn[q] < i0 + e) ? cA + row + sj[q] : sm.sinkA + lane) = gk[q][e] * (bi[e] * dec);
    }
  }
}

// The Gram blocks of tree wave P's tile pair when both tiles are complete (NT = 4, every one of the 8 tiles live):
// tile 7 - P against tiles 0 .. 7 - P, then tile P against 0 .. P, nine blocks as one unrolled sequence, two blocks
// per step. A step's B fragments, masks and gates are read one step ahead, and its products are interleaved with
// the scatter of the previous step's blocks, so the wave issues VALU work while its MFMAs run. The coefficients are
// those of pipe_gram_blocks; two differences in where they go: a non-ancestor entry goes to the sink words at the
// same offset from the sink as the real entry from its row (one select of the offset per entry serves both
// matrices), and a diagonal block also writes a_ii into node i's own slot, which the back substitution never reads
// (step m reads the slots below m of row path(m)).
template <int P, typename S>
__device__ __forceinline__ void pipe_gram_pair(S& sm, const u32x4 (&kf)[2][D / 32], const u32x4 (&qf)[2][D / 32],
                                               int lane) {
  constexpr int NB1 = 8 - P;  // blocks of tile 7 - P (x = 1); then P + 1 blocks of tile P (x = 0)
  constexpr int NB = 9;
  constexpr int KROW = S::KROW;
  const int g4 = lane >> 4, l16 = lane & 15;
  float gi[2][4], bi[2][4];
  int rowoff[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int i0 = (x ? 7 - P : P) * 16 + g4 * 4;
    const f32x4 g = *reinterpret_cast<const f32x4*>(&sm.G[i0]);
    const f32x4 b = *reinterpret_cast<const f32x4*>(&sm.beta[i0]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gi[x][e] = g[e];
      bi[x][e] = b[e];
    }
    rowoff[x] = i0 * CROW;
  }
  static_assert(offsetof(S, sinkP) - offsetof(S, coefP) == offsetof(S, sinkA) - offsetof(S, coefA),
                "each sink must lie at the same distance from its coefficient rows");
  float* const cA = &sm.coefA[0][0];
  const int offP = (int)(&sm.coefP[0][0] - cA);  // a compile-time constant
  float* const sink = &sm.sinkA[0] + lane;
  const uint32_t bit_lo = 1u << l16, bit_hi = bit_lo << 16;

  struct Blk {
    u32x4 bb[D / 32];
    u32x4 mw;
    int sj;
    float gj;
  };
  auto load = [&](int b, Blk& k) __attribute__((always_inline)) {
    const int x = b < NB1 ? 1 : 0;
    const int tp = x ? b : b - NB1;
    const int jn = tp * 16 + l16;
    k.sj = sm.meta.depth[jn] - 1;
    k.gj = sm.G[jn];
    k.mw = *reinterpret_cast<const u32x4*>(&sm.meta.anc[tp >> 1][(x ? 7 - P : P) * 16 + g4 * 4]);
    const uint16_t* br = &sm.kr[jn * KROW + g4 * 8];
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc) k.bb[kc] = *reinterpret_cast<const u32x4*>(br + kc * 32);
  };
  auto scatter = [&](int b, const Blk& k, const f32x4& gk, const f32x4& gq) __attribute__((always_inline)) {
    const int x = b < NB1 ? 1 : 0;
    const int tp = x ? b : b - NB1;
    const uint32_t bit = (tp & 1) ? bit_hi : bit_lo;
    float* const real = cA + rowoff[x] + k.sj;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // the select is on LDS addresses, so that e CROW and the a-to-p distance stay immediate offsets
      float* const dst = (k.mw[e] & bit) != 0 ? real : sink;
      const float dec = __builtin_amdgcn_exp2f(gi[x][e] - k.gj);
      dst[e * CROW] = gk[e] * (bi[x][e] * dec);
      dst[e * CROW + offP] = gq[e] * dec;
    }
  };

  Blk cur[2], nxt[2], prv[2];
  f32x4 gk[2], gq[2], pk[2], pq[2];
  load(0, cur[0]);
  load(1, cur[1]);
#pragma unroll
  for (int s = 0; s < (NB + 1) / 2; ++s) {
    const int b0 = 2 * s;
    const bool two = b0 + 1 < NB;
    if (b0 + 2 < NB) load(b0 + 2, nxt[0]);
    if (b0 + 3 < NB) load(b0 + 3, nxt[1]);
#pragma unroll
    for (int j = 0; j < 2; ++j) gk[j] = gq[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j == 1 && !two) break;
        const int x = b0 + j < NB1 ? 1 : 0;
        const bf16x8 bb = __builtin_bit_cast(bf16x8, cur[j].bb[kc]);
        gk[j] = mfma16(__builtin_bit_cast(bf16x8, kf[x][kc]), bb, gk[j]);
        gq[j] = mfma16(__builtin_bit_cast(bf16x8, qf[x][kc]), bb, gq[j]);
      }
    if (s > 0) {
      scatter(b0 - 2, prv[0], pk[0], pq[0]);
      scatter(b0 - 1, prv[1], pk[1], pq[1]);
      // the next step's LDS reads first, then the MFMAs spread over the step, each followed by a share of the
      // scatter's VALU work and LDS writes
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * (D / 32 + 3), 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i >= (two ? 16 : 8)) break;
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // a step is a scheduling region of its own
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      prv[j] = cur[j];
      if (b0 + 2 + j < NB) cur[j] = nxt[j];
      pk[j] = gk[j];
      pq[j] = gq[j];
    }
  }
  scatter(NB - 1, prv[0], pk[0], pq[0]);  // NB is odd: the last step had one block
}

// max of x over lanes l and l ^ X (X = 16 or 32) by v_permlane16_swap / v_permlane32_swap of x with an opaque copy of
// itself: the two results of a lane are x[l] and x[l ^ X] in some order
template <int X>
__device__ __forceinline__ float half_row_max(float x) {
  int y;
  asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(__builtin_bit_cast(int, x)));
  const auto r = X == 16 ? __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), y, false, false)
                         : __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), y, false, false);
  return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}

// trees of <= 64 nodes (NT <= 2): at most 128 VGPRs, four waves per SIMD, so that two workgroups share a CU (their
// LDS fits twice); 128-node trees: two waves per SIMD, one workgroup per CU
template <int NT, bool CTX>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(NT == 4 ? 2 : 4, NT == 4 ? 2 : 4))) void
tree_gdn_pipe_kernel(GdnArgs a) {
  using S = PipeSmem<NT>;
  constexpr int NMAX = S::NMAX;
  constexpr int NT16 = S::NT16;
  constexpr int KROW = S::KROW;
  constexpr int P = NT;            // tile pairs
  constexpr int TP = 4 / P;        // tree waves per pair (1, 2, 4)
  constexpr int CWC = D / 4;       // value columns of a column wave (32)
  __shared__ S sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4;
  const int l16 = lane & 15;
  const bool treew = w < 4;

  // ---- workgroup -> (request, key head, GQA member): the members of one (request, key head) share the q / k
  //      rows and land on the same XCD (workgroup id modulo 8)
  const int G = a.H / a.HK;
  const int PP = a.R * a.HK;
  const int P8 = (PP + 7) >> 3;
  const int id = blockIdx.x;
  const int rest = id >> 3;
  const int pidx = (rest % P8) * 8 + (id & 7);
  if (pidx >= PP) return;
  const int mem = rest / P8;
  const int r = pidx / a.HK;
  const int hk = pidx % a.HK;
  const int h = hk * G + mem;

  int ns_, n_;
  request_range(a.cu_nodes, r, a.N, ns_, n_);
  const int ns = __builtin_amdgcn_readfirstlane(ns_);
  const int n = __builtin_amdgcn_readfirstlane(n_);
  if (n <= 0) return;
  if (n > NMAX) {
    nan_fill(a.u, a.o, ns, n, a.H, h, 0, D, tid, NTHREADS);
    if (tid == 0 && a.err) atomicOr(a.err, MFD_DEVERR_TOO_MANY_NODES);
    return;
  }
  const int ntiles = (n + 15) >> 4;
  const size_t rh = (size_t)r * a.H + h;
  const int HD = a.H * D, HKD = a.HK * D;
  if (tid < 8) sm.sync[tid] = 0;
  __syncthreads();  // the only workgroup barrier before the last: the counters start at zero
  bool stuck = false;

  if (treew) {
    // ================================ tree waves ================================
    const int p = w % P, tj = w / P;
    const int tile[2] = {p, NT16 - 1 - p};
    const bool live[2] = {tile[0] < ntiles, tile[1] < ntiles};
    const __amdgpu_buffer_rsrc_t rs_k = rsrc(a.k + ((size_t)ns * a.HK + hk) * D, (uint32_t)n * HKD * 2);
    const __amdgpu_buffer_rsrc_t rs_q = rsrc(a.q + ((size_t)ns * a.HK + hk) * D, (uint32_t)n * HKD * 2);
    const int t4 = tid;  // 0 .. 255
    // context (or parents) and gates first, then the K and Q rows of the pair's tiles as 16x16x32 fragments
    // (lane: node 16 t + l16, dims 32 kc + 8 g4 .. + 7); loads are unconditional so that wait counts are static
    constexpr int NCM = (int)(sizeof(TreeMeta<NMAX>) / 16);
    static_assert(NCM <= 512, "two context chunks per tree thread");
    u32x4 cch[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    if constexpr (CTX) {
      const __amdgpu_buffer_rsrc_t rs_c = rsrc(a.ctx + (size_t)r * sizeof(TreeMeta<NMAX>), NCM * 16);
#pragma unroll
      for (int x = 0; x < 2; ++x)
        cch[x] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_c, (uint32_t)(t4 + 256 * x) * 16u, 0, 0));
    }
    // gates: threads 0 .. 127 load g_cum of node t4, threads 128 .. 255 beta of node t4 - 128 (one scattered load
    // per wave, in every tree wave, instead of two in waves 0-1), unconditionally at a clamped node so that no
    // branch makes the wave wait for them before it issues its K / Q rows
    const int gnode = t4 & 127;
    const float gv = (t4 < 128 ? a.g_cum : a.beta)[(size_t)(ns + min(gnode, n - 1)) * a.H + h];
    int par_own = -1;
    if constexpr (!CTX) {
      if (t4 < NMAX && t4 < n) par_own = parent_of(a.parents, a.anc8, ns, t4, n);
    }
    u32x4 kf[2][D / 32], qf[2][D / 32];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const uint32_t off = (uint32_t)((tile[x] * 16 + l16) * HKD + g4 * 8) * 2u;
#pragma unroll
      for (int kc = 0; kc < D / 32; ++kc) {
        kf[x][kc] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_k, off + kc * 64, 0, 0));
        qf[x][kc] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_q, off + kc * 64, 0, 0));
      }
    }
    if (t4 < NMAX) {
      const float g_own = t4 < n ? gv : 0.f;
      if constexpr (!CTX) sm.par[t4] = par_own;
      sm.G[t4] = g_own * 1.44269504088896341f;  // log2(e): the Gram's decays are exp2 of differences
      sm.eG[t4] = t4 < n ? __expf(g_own) : 0.f;
      sm.rexp[0][t4] = 0;
      sm.rexp[1][t4] = 0;
    } else if (t4 >= 128 && gnode < NMAX) {
      sm.beta[gnode] = gnode < n ? gv : 0.f;
    }
    if constexpr (CTX) {
#pragma unroll
      for (int x = 0; x < 2; ++x)
        if (t4 + 256 * x < NCM) reinterpret_cast<u32x4*>(&sm.meta)[t4 + 256 * x] = cch[x];
    } else {
      if (t4 == 0) sm.meta.bad = 0;
    }
    if (tj == 0) {  // the K and Q rows into LDS: the Gram blocks' second operand, the column waves' R and E
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        uint16_t* krow = &sm.kr[(tile[x] * 16 + l16) * KROW + g4 * 8];
        uint16_t* qrow = &sm.qr[(tile[x] * 16 + l16) * KROW + g4 * 8];
#pragma unroll
        for (int kc = 0; kc < D / 32; ++kc) {
          *reinterpret_cast<u32x4*>(krow + kc * 32) = kf[x][kc];
          *reinterpret_cast<u32x4*>(qrow + kc * 32) = qf[x][kc];
        }
      }
    }
    bool tree_ok = true;
    group_signal(&sm.sync[PS_TREE]);  // K / Q rows and gates (the column waves start their loads on this)
    stuck |= !group_wait(&sm.sync[PS_TREE], 4);
    if constexpr (!CTX) {
      if (t4 < NMAX) walk_root_path(sm.meta, sm.par, t4, n);
      group_signal(&sm.sync[PS_TREE]);
      stuck |= !group_wait(&sm.sync[PS_TREE], 8);  // every root path
    } else {
      if (sm.meta.n != n || sm.meta.nmax != NMAX) {  // a context built for another request size or max_nodes
        tree_ok = false;
        if (t4 == 0) atomicOr(&sm.meta.bad, MFD_DEVERR_BAD_CONTEXT);
      }
    }
    // a rejected tree: the tree phases are skipped (its paths are not usable); the hand-overs still happen, and
    // the outputs are replaced by NaN at the end
    tree_ok = tree_ok && sm.meta.bad == 0;
    stuck |= !group_wait(&sm.sync[PS_CLEAR], 4);  // coefficient rows and staged rows cleared

    // ---- Gram blocks (t, t') for the pair's tiles t and t' <= t, four at a time: the pair's tree waves take blocks
    //      tj, tj + TP, ... of each tile
    if (tree_ok) {
      bool done = false;
      if constexpr (NT == 4) {
        if (ntiles == NT16) {  // both tiles of every pair complete: one pipelined sequence per wave
          switch (p) {
            case 0: pipe_gram_pair<0>(sm, kf, qf, lane); break;
            case 1: pipe_gram_pair<1>(sm, kf, qf, lane); break;
            case 2: pipe_gram_pair<2>(sm, kf, qf, lane); break;
            default: pipe_gram_pair<3>(sm, kf, qf, lane); break;
          }
          done = true;
        }
      }
      if (!done) {
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          if (!live[x]) continue;
          const int t = tile[x];
          // NT blocks per call: with NT < 4 a wave has at most NT blocks of a tile (TP = 4 / NT waves share it), so
          // no call computes products of blocks it does not keep
          for (int tp = tj; tp <= t; tp += NT * TP) pipe_gram_blocks<NT>(sm, kf[x], qf[x], t, tp, TP, min(NT, (t - tp) / TP + 1), lane);
        }
      }
    }
    group_signal(&sm.sync[PS_COEF]);
    stuck |= !group_wait(&sm.sync[PS_COEF], 4);  // every node's coefficient rows

    // ---- rows of T (x L = e_{d-1}) and W (x L = p_i), L = I + A on the root path (L[m][s] = a_{path(m)}[s]),
    //      right-looking over the path with the a rows of the next two steps read ahead; into LDS as fp16
    //      scaled by 2^-e, the largest entry in [1/2, 1) (job: node, matrix)
    {
      const int job = lane * TP + tj;
      const int kind = job >> 5;
      const int qs = job & 31;
      // NT = 4: wave w takes the rows of tiles 2 w and 2 w + 1 (not its Gram pair), so that the shallow low tiles
      // are staged first (the steps past a wave's deepest path are skipped) and published tile pair by tile pair;
      // otherwise the rows of the wave's Gram pair. (Masked to NMAX - 1, which it never exceeds: the compiler then
      // knows the path entries and row offsets are small and forms them with 24-bit multiplies.)
      const int ta = NT == 4 ? 2 * w : tile[0], tb = NT == 4 ? 2 * w + 1 : tile[1];
      const int i = (qs < 16 ? ta * 16 + qs : tb * 16 + qs - 16) & (NMAX - 1);
      if (tree_ok && job < 64 && i < n) {
        const int dep = sm.meta.depth[i];
        int pth[MAXD];
        float rhs[MAXD], acc[MAXD], X[MAXD];
#pragma unroll
        for (int s4 = 0; s4 < MAXD; s4 += 4) {
          const uint32_t pw = *reinterpret_cast<const uint32_t*>(&sm.meta.path[i][s4]);
          const f32x4 xp = *reinterpret_cast<const f32x4*>(&sm.coefP[i][s4]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pth[s4 + e] = (s4 + e < dep) ? (int)((pw >> (8 * e)) & 0xFFu) : i;
            rhs[s4 + e] = kind ? xp[e] : ((s4 + e == dep - 1) ? 1.f : 0.f);
            acc[s4 + e] = 0.f;
          }
        }
        // NT = 4: the deepest root path among the wave's active jobs (binary search over ballots; depths are
        // <= MAXD); smaller trees run every step (the search and the step branches cost them more than they save)
        int md = MAXD;
        if constexpr (NT == 4) {
          md = 0;
#pragma unroll
          for (int b = 4; b >= 0; --b) {
            const int cand = md | (1 << b);
            if (cand <= MAXD && __builtin_amdgcn_ballot_w64(dep >= cand) != 0) md = cand;
          }
        }
        // the a rows of steps m, m - 1 and m - 2 (step m reads slots s < m of row path(m))
        f32x4 r0[MAXD / 4], r1[MAXD / 4], r2[MAXD / 4];
#pragma unroll
        for (int s4 = 0; s4 < MAXD - 1; s4 += 4) r0[s4 / 4] = *reinterpret_cast<const f32x4*>(&sm.coefA[pth[MAXD - 1]][s4]);
#pragma unroll
        for (int s4 = 0; s4 < MAXD - 2; s4 += 4) r1[s4 / 4] = *reinterpret_cast<const f32x4*>(&sm.coefA[pth[MAXD - 2]][s4]);
#pragma unroll
        for (int m = MAXD - 1; m >= 0; --m) {
          if (m > 2) {
#pragma unroll
            for (int s4 = 0; s4 < m - 2; s4 += 4) r2[s4 / 4] = *reinterpret_cast<const f32x4*>(&sm.coefA[pth[m - 2]][s4]);
          }
          // steps at or past the deepest path of the wave's jobs (md, wave-uniform) have x = 0 on every lane: their
          // products are skipped
          if (m < md) {
            const float xm = m < dep ? rhs[m] - acc[m] : 0.f;
            X[m] = xm;
#pragma unroll
            for (int s4 = 0; s4 < m; s4 += 4)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (s4 + e < m) acc[s4 + e] = fmaf(xm, r0[s4 / 4][e], acc[s4 + e]);
          } else {
            X[m] = 0.f;
          }
#pragma unroll
          for (int s4 = 0; s4 < m - 1; s4 += 4) r0[s4 / 4] = r1[s4 / 4];
#pragma unroll
          for (int s4 = 0; s4 < m - 2; s4 += 4) r1[s4 / 4] = r2[s4 / 4];
        }
        float mx = 0.f;
#pragma unroll
        for (int s = 0; s < MAXD; ++s) mx = fmaxf(mx, fabsf(X[s]));
        const int ex = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) : 0;
        const int t = i >> 4;
        _Float16* row = reinterpret_cast<_Float16*>(&sm.st[kind][S::soff(t) + (i & 15) * S::srow(t)]);
#pragma unroll
        for (int s = 0; s < MAXD; ++s)
          if (s < dep) row[stage_pos(pth[s])] = (_Float16)__builtin_ldexpf(X[s], -ex);
        sm.rexp[kind][i] = ex;
      }
    }
    if constexpr (NT == 4) group_signal(&sm.sync[PS_TWT + w]);
    else group_signal(&sm.sync[PS_TW]);
  } else {
    // ================================ column waves ================================
    const int cw = w - 4;
    const int cb = cw * CWC;
    const int c4 = tid - 256;  // 0 .. 255
    // clears of the coefficient and staged rows (the tree waves' targets)
    {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      for (int x = c4; x < NMAX * CROW / 4; x += 256) {
        reinterpret_cast<f32x4*>(&sm.coefA[0][0])[x] = z;
        reinterpret_cast<f32x4*>(&sm.coefP[0][0])[x] = z;
      }
      const u32x4 zz = {0u, 0u, 0u, 0u};
      for (int x = c4; x < 2 * S::STAGE / 8; x += 256) reinterpret_cast<u32x4*>(&sm.st[0][0])[x] = zz;
    }
    group_signal(&sm.sync[PS_CLEAR]);
    // S0 as the B fragments of K S0 (and the A fragments of S0^T Q^T): lane l loads column cb + 16 ct + l16 at
    // k = 32 kc + 8 g4 .. + 7 one value at a time (each load of the wave reads four 64-byte row pieces), so the
    // fragments need no transpose once they land. Then the v rows of this wave's columns as 16x16x32 fragments
    // (lane: node 16 t + l16, columns cb + 8 g4 .. + 7).
    const __amdgpu_buffer_rsrc_t rs_s0 = rsrc(a.s0 + rh * D * D, D * D * 4);
    const __amdgpu_buffer_rsrc_t rs_v = rsrc(a.v + ((size_t)ns * a.H + h) * D, (uint32_t)n * HD * 2);
    float s0v[2][D / 32][8];
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t off = (uint32_t)((kc * 32 + g4 * 8 + j) * D + cb + ct * 16 + l16) * 4u;
          s0v[ct][kc][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_s0, off, 0, 0));
        }
    u32x4 vf[NT16];
#pragma unroll
    for (int t = 0; t < NT16; ++t)
      vf[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
          rs_v, (uint32_t)((t * 16 + l16) * HD + cb + g4 * 8) * 2u, 0, 0));
    // S0 in bf16 (rounded to nearest even, as the reference's s_blk)
    bf16x8 sa[2][D / 32];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int kc = 0; kc < D / 32; ++kc) {
        u32x4 pk;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          pk[jj] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){s0v[ct][kc][2 * jj], s0v[ct][kc][2 * jj + 1]}, bf16x2));
        sa[ct][kc] = __builtin_bit_cast(bf16x8, pk);
      }
    stuck |= !group_wait(&sm.sync[PS_TREE], 4);  // K / Q rows and gates
    // R = beta (v - e^G K S0) for every node and this wave's 32 columns, in the C layout of A = K rows (from LDS),
    // B = S0 fragments: lane l holds column cb + 16 ct + l16 of nodes 16 t + 4 g4 .. + 3. v reaches that layout
    // through one MFMA against an identity block per tile and column tile.
    bf16x8 eye[2];  // B fragments of the column selections [16 ct, 16 ct + 16) of a 32-column v fragment
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int e = 0; e < 8; ++e) eye[ct][e] = (__bf16)((g4 * 8 + e == ct * 16 + l16) ? 1.f : 0.f);
    f32x4 rr[NT16][2];
#pragma unroll
    for (int t = 0; t < NT16; ++t)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) rr[t][ct] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // two tiles at a time (four accumulation chains; fragments read just ahead of their products). NT = 4: every
    // tile, live or not, in one branch-free sequence, so that the reads of later tiles overlap the products of
    // earlier ones: the K rows and v values of nodes past n are zeros (buffer loads past the range return 0) and so
    // is their beta, which makes their R zero. Smaller trees (often ragged, with few live tiles) skip dead tiles.
#pragma unroll
    for (int t = 0; t < NT16; t += 2) {
      if constexpr (NT < 4) {
        if (t >= ntiles) break;
      }
#pragma unroll
      for (int kc = 0; kc < D / 32; ++kc) {
        const bf16x8 k0 = ld_lds8(&sm.kr[(t * 16 + l16) * KROW + kc * 32 + g4 * 8]);
        const bf16x8 k1 = ld_lds8(&sm.kr[(t * 16 + 16 + l16) * KROW + kc * 32 + g4 * 8]);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          rr[t][ct] = mfma16(k0, sa[ct][kc], rr[t][ct]);
          rr[t + 1][ct] = mfma16(k1, sa[ct][kc], rr[t + 1][ct]);
        }
      }
    }
    float cm[2] = {0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NT16; ++t) {
      const f32x4 bi = *reinterpret_cast<const f32x4*>(&sm.beta[t * 16 + g4 * 4]);
      const f32x4 ei = *reinterpret_cast<const f32x4*>(&sm.eG[t * 16 + g4 * 4]);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const f32x4 vt = (NT == 4 || t < ntiles)
                             ? mfma16(__builtin_bit_cast(bf16x8, vf[t]), eye[ct], (f32x4){0.f, 0.f, 0.f, 0.f})
                             : (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          rr[t][ct][e] = bi[e] * (vt[e] - ei[e] * rr[t][ct][e]);
          cm[ct] = fmaxf(cm[ct], fabsf(rr[t][ct][e]));
        }
      }
    }
    // per-column scale 2^-e (the column's largest |R| in [1/2, 1)); every node of the column is in this wave,
    // spread over the four lane groups
    int ce[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      // max over lanes l, l ^ 16, l ^ 32, l ^ 48 by two lane-row swaps (no LDS round trip)
      float m = half_row_max<16>(cm[ct]);
      m = half_row_max<32>(m);
      ce[ct] = m > 0.f ? __builtin_amdgcn_frexp_expf(m) : 0;
      if (g4 == 0) sm.cexp[cb + ct * 16 + l16] = ce[ct];
    }
    // the scaled fp16 R pairs; in the A layout of R^T for chunk kc (tiles 2 kc and 2 kc + 1, rows 4 g4 .. + 3 of
    // each), which orders the nodes of a 32-node chunk as stage_pos does
    uint32_t rh2[NT16][2][2];
#pragma unroll
    for (int t = 0; t < NT16; ++t)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const float s = __builtin_ldexpf(1.f, -ce[ct]);
        const f16x2 lo = __builtin_convertvector((f32x2){rr[t][ct][0] * s, rr[t][ct][1] * s}, f16x2);
        const f16x2 hi = __builtin_convertvector((f32x2){rr[t][ct][2] * s, rr[t][ct][3] * s}, f16x2);
        rh2[t][ct][0] = __builtin_bit_cast(uint32_t, lo);
        rh2[t][ct][1] = __builtin_bit_cast(uint32_t, hi);
      }
    // ---- per tile: E^T = e^G S0^T Q^T (C register e of lane l: column cb + 16 ct + 4 g4 + e, node 16 t + l16;
    //      A = the S0 fragments, B = Q rows), u^T = R^T T^T and o^T = E^T + R^T W^T over the k chunks (32 nodes)
    //      up to the tile's own (A = R from registers, B = the staged T / W rows), unscaled by
    //      2^{eT(node) + eR(col)} and 2^{eW(node) + eR(col)}. E is computed here, once T and W are staged, so
    //      that its accumulators need not be held: these products hide behind the stores.
    f16x8 ra[2][NMAX / 32];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int kc = 0; kc < NMAX / 32; ++kc) {
        const u32x4 pk = {rh2[2 * kc][ct][0], rh2[2 * kc][ct][1], rh2[2 * kc + 1][ct][0], rh2[2 * kc + 1][ct][1]};
        ra[ct][kc] = __builtin_bit_cast(f16x8, pk);
      }
    int cexc[2][4];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int4 c4v = *reinterpret_cast<const int4*>(&sm.cexp[cb + ct * 16 + g4 * 4]);
      cexc[ct][0] = c4v.x; cexc[ct][1] = c4v.y; cexc[ct][2] = c4v.z; cexc[ct][3] = c4v.w;
    }
    if constexpr (NT != 4) stuck |= !group_wait(&sm.sync[PS_TW], 4);  // T and W rows of every node
    const __amdgpu_buffer_rsrc_t rs_u = rsrc(a.u + ((size_t)ns * a.H + h) * D, (uint32_t)n * HD * 4);
    const __amdgpu_buffer_rsrc_t rs_o = rsrc(a.o + ((size_t)ns * a.H + h) * D, (uint32_t)n * HD * 4);
#pragma unroll
    for (int t = 0; t < NT16; ++t) {
      if (t >= ntiles) break;
      // NT = 4: the T and W rows of tiles t and t + 1 come from tree wave t / 2
      if constexpr (NT == 4) {
        if ((t & 1) == 0) stuck |= !group_wait(&sm.sync[PS_TWT + (t >> 1)], 1);
      }
      const int nd = t * 16 + l16;
      const int eT = sm.rexp[0][nd];
      const int eW = sm.rexp[1][nd];
      const float eg = sm.eG[nd];
      f32x4 ee[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int kc = 0; kc < D / 32; ++kc) {
        const bf16x8 qb = ld_lds8(&sm.qr[nd * KROW + kc * 32 + g4 * 8]);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) ee[ct] = mfma16(sa[ct][kc], qb, ee[ct]);
      }
      f32x4 au[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
      f32x4 ao[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) ao[ct][e] = __builtin_ldexpf(ee[ct][e] * eg, -(eW + cexc[ct][e]));
      const uint16_t* sbT = &sm.st[0][S::soff(t) + l16 * S::srow(t) + g4 * 8];
      const uint16_t* sbW = &sm.st[1][S::soff(t) + l16 * S::srow(t) + g4 * 8];
#pragma unroll
      for (int kc = 0; kc <= (t >> 1); ++kc) {
        const f16x8 bt = __builtin_bit_cast(f16x8, *reinterpret_cast<const u16x8*>(sbT + kc * 32));
        const f16x8 bw = __builtin_bit_cast(f16x8, *reinterpret_cast<const u16x8*>(sbW + kc * 32));
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          au[ct] = mfma16_f16(ra[ct][kc], bt, au[ct]);
          ao[ct] = mfma16_f16(ra[ct][kc], bw, ao[ct]);
        }
      }
      const uint32_t st_off = (uint32_t)(nd * HD + cb + g4 * 4) * 4u;
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        store4(rs_u, st_off + ct * 64, __builtin_ldexpf(au[ct][0], eT + cexc[ct][0]),
               __builtin_ldexpf(au[ct][1], eT + cexc[ct][1]), __builtin_ldexpf(au[ct][2], eT + cexc[ct][2]),
               __builtin_ldexpf(au[ct][3], eT + cexc[ct][3]));
        store4(rs_o, st_off + ct * 64, __builtin_ldexpf(ao[ct][0], eW + cexc[ct][0]),
               __builtin_ldexpf(ao[ct][1], eW + cexc[ct][1]), __builtin_ldexpf(ao[ct][2], eW + cexc[ct][2]),
               __builtin_ldexpf(ao[ct][3], eW + cexc[ct][3]));
      }
    }
  }
  // a rejected tree or a hand-over wait that ran out: this workgroup's outputs become NaN (never silent)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores have completed
  const int bad = __syncthreads_or(stuck ? 1 : 0);
  const int tbad = sm.meta.bad;
  if (bad || tbad) {
    nan_fill(a.u, a.o, ns, n, a.H, h, 0, D, tid, NTHREADS);
    if (tid == 0 && a.err) atomicOr(a.err, tbad | (bad ? MFD_DEVERR_INTERNAL : 0));
  }
}

// One workgroup per request: the tree context block of the request (walk of every node's root path).
template <int NT>
__global__ __launch_bounds__(128) void tree_ctx_kernel(const int32_t* parents, const int8_t* anc8,
                                                       const int32_t* cu_nodes, int N, uint8_t* ctx, int32_t* err) {
  constexpr int NMAX = 32 * NT;
  __shared__ TreeMeta<NMAX> m;
  __shared__ int par[NMAX];
  const int tid = threadIdx.x;
  const int r = blockIdx.x;
  int ns, n;
  request_range(cu_nodes, r, N, ns, n);
  const bool fits = n <= NMAX;
  if (tid == 0) {
    m.bad = fits ? 0 : MFD_DEVERR_TOO_MANY_NODES;
    m.n = n;
    m.nmax = NMAX;
    m.pad = 0;
  }
  if (tid < NMAX) par[tid] = (fits && tid < n) ? parent_of(parents, anc8, ns, tid, n) : -1;
  __syncthreads();
  if (tid < NMAX) walk_root_path(m, par, tid, fits ? n : 0);
  __syncthreads();
  if (tid == 0 && m.bad && err) atomicOr(err, m.bad);
  constexpr int NCM = (int)(sizeof(TreeMeta<NMAX>) / 16);
  const uint4* src = reinterpret_cast<const uint4*>(&m);
  uint4* dst = reinterpret_cast<uint4*>(ctx + (size_t)r * sizeof(TreeMeta<NMAX>));
  for (int c = tid; c < NCM; c += 128) dst[c] = src[c];
}

size_t ctx_block_bytes(int max_nodes) {
  if (max_nodes <= 32) return sizeof(TreeMeta<32>);
  if (max_nodes <= 64) return sizeof(TreeMeta<64>);
  if (max_nodes <= FUSED_MAX_NODES) return sizeof(TreeMeta<128>);
  return gdn_large_ctx_block_bytes(max_nodes);
}

template <int NT>
int launch_gdn(const GdnArgs& args, hipStream_t stream) {
  const int G = args.H / args.HK;
  const int P = args.R * args.HK;
  const int P8 = (P + 7) / 8;
  const dim3 grid(8 * P8 * G * args.csplit);
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(NTHREADS), 0, stream, args); };
  if (args.csplit == 1) {  // grids that fill the chip: the phase-ordered kernel
    if (args.ctx)
      go(tree_gdn_pipe_kernel<NT, true>);
    else
      go(tree_gdn_pipe_kernel<NT, false>);
  } else if (args.ctx) {
    if (args.csplit == 4) go(tree_gdn_kernel<NT, true, 4>);
    else if (args.csplit == 2) go(tree_gdn_kernel<NT, true, 2>);
    else go(tree_gdn_kernel<NT, true, 1>);
  } else {
    if (args.csplit == 4) go(tree_gdn_kernel<NT, false, 4>);
    else if (args.csplit == 2) go(tree_gdn_kernel<NT, false, 2>);
    else go(tree_gdn_kernel<NT, false, 1>);
  }
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

int launch_gdn_fused(const GdnArgs& args_in, int max_nodes, hipStream_t s) {
  GdnArgs args = args_in;
  // a grid of (request, value head) units that fills at most a quarter (a half) of the CUs splits each
  // unit's value columns over 4 (2) workgroups: the tree part is computed by each of them, the S0 loads,
  // S0 products and u / o stores are shared out
  const int64_t units = (int64_t)args.R * args.H;
  const int cus = mfd_num_cus();
  args.csplit = units * 4 <= cus ? 4 : (units * 2 <= cus ? 2 : 1);
  if (max_nodes <= 32) return launch_gdn<1>(args, s);
  if (max_nodes <= 64) return launch_gdn<2>(args, s);
  return launch_gdn<4>(args, s);
}

constexpr int64_t WS_ALIGN = 256;
int64_t align_up(int64_t x) { return (x + WS_ALIGN - 1) / WS_ALIGN * WS_ALIGN; }
// Gram rows of the large-tree path: [N][HK][2][MAXD] f32
int64_t gram_bytes(int N, int HK) { return (int64_t)N * HK * 2 * MAXD * 4; }

// Workspace of the large-tree path: the tree contexts (when the call builds them) then the Gram rows.
int64_t gdn_workspace_bytes(int R, int N, int HK, int max_nodes, bool has_ctx) {
  if (max_nodes <= FUSED_MAX_NODES) return 0;
  const int64_t c = has_ctx ? 0 : align_up((int64_t)R * (int64_t)gdn_large_ctx_block_bytes(max_nodes));
  return c + align_up(gram_bytes(N, HK));
}

// Argument checks shared by the GDN entry points; returns MFD_OK or the error already recorded.
int check_gdn_args(const char* fn, int R, int N, int HK, int H, int D_, int max_nodes, const int32_t* cu_nodes) {
  if (D_ != D) return mfd_set_error(MFD_ERR_UNSUPPORTED, "%s: head dim %d (only %d)", fn, D_, D);
  if (R < 1 || N < 0 || HK < 1 || H < 1 || H % HK != 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "%s: bad sizes R=%d N=%d HK=%d H=%d", fn, R, N, HK, H);
  if (!cu_nodes && R != 1) return mfd_set_error(MFD_ERR_INVALID_ARG, "%s: cu_nodes required for R > 1", fn);
  if (max_nodes < 0 || max_nodes > MFD_GDN_MAX_NODES)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "%s: max_nodes %d exceeds %d", fn, max_nodes, MFD_GDN_MAX_NODES);
  if (!cu_nodes && N > max_nodes) return mfd_set_error(MFD_ERR_INVALID_ARG, "%s: N=%d > max_nodes=%d", fn, N, max_nodes);
  return MFD_OK;
}

int check_workspace(const char* fn, void* ws, int64_t ws_bytes, int64_t need) {
  if (need == 0) return MFD_OK;
  if (!ws || ws_bytes < need || ((uintptr_t)ws & (WS_ALIGN - 1)) != 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "%s: workspace of %lld bytes (256-byte aligned) required, got %lld",
                         fn, (long long)need, (long long)(ws ? ws_bytes : 0));
  return MFD_OK;
}

int build_context(const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R, int N, int max_nodes,
                  uint8_t* c, int32_t* err_flag, hipStream_t s) {
  if (max_nodes > FUSED_MAX_NODES) return gdn_large_context(parents, anc8, cu_nodes, R, N, max_nodes, c, err_flag, s);
  if (max_nodes <= 32)
    hipLaunchKernelGGL(tree_ctx_kernel<1>, dim3(R), dim3(128), 0, s, parents, anc8, cu_nodes, N, c, err_flag);
  else if (max_nodes <= 64)
    hipLaunchKernelGGL(tree_ctx_kernel<2>, dim3(R), dim3(128), 0, s, parents, anc8, cu_nodes, N, c, err_flag);
  else
    hipLaunchKernelGGL(tree_ctx_kernel<4>, dim3(R), dim3(128), 0, s, parents, anc8, cu_nodes, N, c, err_flag);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

// Large-tree path: (tree contexts) + Gram rows + the main kernel; ctx given or built into the workspace.
int run_large_path(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum, const float* beta,
                   const float* s0, const int32_t* parents, const int8_t* anc8, const uint8_t* ctx,
                   const int32_t* cu_nodes, int R, int N, int HK, int H, int max_nodes, float* u, float* o,
                   int32_t* err_flag, void* ws, hipStream_t s) {
  uint8_t* w = static_cast<uint8_t*>(ws);
  if (!ctx) {
    if (int rc = gdn_large_context(parents, anc8, cu_nodes, R, N, max_nodes, w, err_flag, s)) return rc;
    ctx = w;
    w += align_up((int64_t)R * (int64_t)gdn_large_ctx_block_bytes(max_nodes));
  }
  GdnLargeArgs la{q, k, v, g_cum, beta, s0, cu_nodes, ctx, reinterpret_cast<float*>(w), u, o, err_flag, R, N, HK, H};
  return gdn_large_run(la, max_nodes, s);
}

}  // namespace

extern "C" int64_t mfd_tree_gdn_workspace_bytes(int R, int N, int HK, int max_nodes, int has_ctx) {
  if (R < 1 || N < 0 || HK < 1 || max_nodes < 0 || max_nodes > MFD_GDN_MAX_NODES) return -1;
  return gdn_workspace_bytes(R, N, HK, max_nodes, has_ctx != 0);
}

namespace {
// Shared body of mfd_tree_gdn and mfd_tree_gdn_noalloc; the workspace is checked by the caller.
int tree_gdn_impl(const char* fn, const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum,
                  const float* beta, const float* s0, const int32_t* parents, const int8_t* anc8,
                  const int32_t* cu_nodes, int R, int N, int HK, int H, int max_nodes, float* u, float* o,
                  int32_t* err_flag, void* workspace, hipStream_t s) {
  if (max_nodes > FUSED_MAX_NODES)
    return run_large_path(q, k, v, g_cum, beta, s0, parents, anc8, nullptr, cu_nodes, R, N, HK, H, max_nodes, u, o,
                          err_flag, workspace, s);
  (void)fn;
  GdnArgs args{q, k, v, g_cum, beta, s0, parents, anc8, cu_nodes, nullptr, u, o, err_flag, R, N, HK, H};
  return launch_gdn_fused(args, max_nodes, s);
}

int check_tree_gdn_call(const char* fn, const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum,
                        const float* beta, const float* s0, const int32_t* parents, const int8_t* anc8,
                        const int32_t* cu_nodes, int R, int N, int HK, int H, int D_, int max_nodes, float* u,
                        float* o) {
  if (int rc = check_gdn_args(fn, R, N, HK, H, D_, max_nodes, cu_nodes)) return rc;
  if (!parents && (!anc8 || R != 1))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "%s: parents required unless R == 1 and anc8 given", fn);
  if (N == 0 || max_nodes == 0) return MFD_OK;
  if (!q || !k || !v || !g_cum || !beta || !s0 || !u || !o)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "%s: null tensor pointer", fn);
  return MFD_OK;
}
}  // namespace

extern "C" int mfd_tree_gdn(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum,
                            const float* beta, const float* s0, const int32_t* parents, const int8_t* anc8,
                            const int32_t* cu_nodes, int R, int N, int HK, int H, int D_, int max_nodes, float* u,
                            float* o, int32_t* err_flag, void* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = check_tree_gdn_call("mfd_tree_gdn", q, k, v, g_cum, beta, s0, parents, anc8, cu_nodes, R, N, HK, H,
                                   D_, max_nodes, u, o))
    return rc;
  if (N == 0 || max_nodes == 0) return MFD_OK;
  const int64_t need = gdn_workspace_bytes(R, N, HK, max_nodes, false);
  if (int rc = check_workspace("mfd_tree_gdn", workspace, workspace_bytes, need)) return rc;
  return tree_gdn_impl("mfd_tree_gdn", q, k, v, g_cum, beta, s0, parents, anc8, cu_nodes, R, N, HK, H, max_nodes, u,
                       o, err_flag, workspace, static_cast<hipStream_t>(stream));
}

// ---- allocation-free variant (no counterpart in the reference): for callers that cannot allocate (code under
//      graph capture, serving loops that forbid hipMalloc). The large-tree path's workspace (tree contexts and
//      Gram rows) lives in this file-scope device array; every GPU the library runs on holds its own copy until
//      the process ends. The kernels write every byte they later read (contexts and Gram rows are written whole
//      before use), so nothing needs clearing between calls; calls that overlap on one GPU share the array and
//      race.
static __device__ __align__(256) uint8_t scratch[MFD_GDN_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};  // device address of `scratch` on each device, looked up once

// Address of this device's copy of `scratch` (the current device: the caller's stream must belong to it).
int current_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mfd_set_hip_error(e);
  if (dev < 0 || dev >= MAX_DEVICES)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_tree_gdn_noalloc: device %d beyond %d", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return mfd_set_hip_error(e);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MFD_OK;
}
}  // namespace

extern "C" int mfd_tree_gdn_noalloc(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum,
                                    const float* beta, const float* s0, const int32_t* parents, const int8_t* anc8,
                                    const int32_t* cu_nodes, int R, int N, int HK, int H, int D_, int max_nodes,
                                    float* u, float* o, int32_t* err_flag, void* stream) {
  const char* fn = "mfd_tree_gdn_noalloc";
  if (int rc = check_tree_gdn_call(fn, q, k, v, g_cum, beta, s0, parents, anc8, cu_nodes, R, N, HK, H, D_, max_nodes,
                                   u, o))
    return rc;
  if (N == 0 || max_nodes == 0) return MFD_OK;
  const int64_t need = gdn_workspace_bytes(R, N, HK, max_nodes, false);
  if (need > (int64_t)MFD_GDN_SCRATCH_BYTES)
    return mfd_set_error(MFD_ERR_UNSUPPORTED,
                         "%s: R=%d N=%d HK=%d max_nodes=%d need %lld bytes of scratch, the static scratch holds %lld",
                         fn, R, N, HK, max_nodes, (long long)need, (long long)MFD_GDN_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0)
    if (int rc = current_scratch(&ws)) return rc;
  return tree_gdn_impl(fn, q, k, v, g_cum, beta, s0, parents, anc8, cu_nodes, R, N, HK, H, max_nodes, u, o, err_flag,
                       ws, static_cast<hipStream_t>(stream));
}

extern "C" size_t mfd_tree_ctx_bytes(int R, int max_nodes) {
  if (R < 1 || max_nodes < 1 || max_nodes > MFD_GDN_MAX_NODES) return 0;
  return (size_t)R * ctx_block_bytes(max_nodes);
}

extern "C" int mfd_tree_context(const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R, int N,
                                int max_nodes, void* ctx, int64_t ctx_bytes, int32_t* err_flag, void* stream) {
  if (R < 1 || N < 0) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_context: bad sizes R=%d N=%d", R, N);
  if (!cu_nodes && R != 1) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_context: cu_nodes required for R > 1");
  if (!parents && (!anc8 || R != 1))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_context: parents required unless R == 1 and anc8 given");
  if (max_nodes < 1 || max_nodes > MFD_GDN_MAX_NODES)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_tree_context: max_nodes %d not in [1, %d]", max_nodes,
                         MFD_GDN_MAX_NODES);
  if (!ctx || ((uintptr_t)ctx & 15) != 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_context: ctx must be a 16-byte aligned device buffer");
  if (ctx_bytes < (int64_t)mfd_tree_ctx_bytes(R, max_nodes))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_context: ctx of %lld bytes, %lld needed", (long long)ctx_bytes,
                         (long long)mfd_tree_ctx_bytes(R, max_nodes));
  return build_context(parents, anc8, cu_nodes, R, N, max_nodes, static_cast<uint8_t*>(ctx), err_flag,
                       static_cast<hipStream_t>(stream));
}

extern "C" int mfd_tree_gdn_ctx(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g_cum,
                                const float* beta, const float* s0, const void* ctx, int64_t ctx_bytes,
                                const int32_t* cu_nodes, int R, int N, int HK, int H, int D_, int max_nodes, float* u,
                                float* o, int32_t* err_flag, void* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = check_gdn_args("mfd_tree_gdn_ctx", R, N, HK, H, D_, max_nodes, cu_nodes)) return rc;
  if (!ctx || ((uintptr_t)ctx & 15) != 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gdn_ctx: ctx must be a 16-byte aligned device buffer");
  if (N == 0 || max_nodes == 0) return MFD_OK;
  // the context must hold R blocks of the layout this max_nodes selects (the kernels read them in full)
  if (ctx_bytes < (int64_t)mfd_tree_ctx_bytes(R, max_nodes))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gdn_ctx: ctx of %lld bytes, %lld needed for R=%d max_nodes=%d",
                         (long long)ctx_bytes, (long long)mfd_tree_ctx_bytes(R, max_nodes), R, max_nodes);
  if (!q || !k || !v || !g_cum || !beta || !s0 || !u || !o)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gdn_ctx: null tensor pointer");
  const int64_t need = gdn_workspace_bytes(R, N, HK, max_nodes, true);
  if (int rc = check_workspace("mfd_tree_gdn_ctx", workspace, workspace_bytes, need)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (max_nodes > FUSED_MAX_NODES)
    return run_large_path(q, k, v, g_cum, beta, s0, nullptr, nullptr, static_cast<const uint8_t*>(ctx), cu_nodes, R,
                          N, HK, H, max_nodes, u, o, err_flag, workspace, s);
  GdnArgs args{q, k, v, g_cum, beta, s0, nullptr, nullptr, cu_nodes, static_cast<const uint8_t*>(ctx), u, o,
               err_flag, R, N, HK, H};
  return launch_gdn_fused(args, max_nodes, s);
}
