// Tree gated-delta-rule verification of trees above 128 nodes (up to MFD_GDN_MAX_NODES), gfx950.
//
// Same quantities as the fused kernel (tree_gdn.hip; inference/hf/tree_gdn_kernel.py:3-6,
// inference/hf/qwen35_tree.py:9-20): for the nodes of one tree in topological order,
//   u = (I + A)^{-1} R,  R_i = beta_i (v_i - e^{G_i} S0^T k_i),   A_ij = beta_i e^{G_i-G_j} k_i.k_j (strict anc.)
//   o = E + P u,         E_i = e^{G_i} S0^T q_i,                  P_ij = e^{G_i-G_j} q_i.k_j   (anc. or self)
// The fused kernel holds a whole tree's K / Q / v rows in LDS, which a 512-node tree does not fit. Here every
// tree quantity is kept per root-path slot (a node has at most MAXD ancestors-or-self), so the work and the LDS
// footprint grow linearly in the node count:
//   tree_ctx_large_kernel   one workgroup per request: each node's root path (node ids by depth) and depth
//   tree_gram_kernel        one workgroup per (request, key head, 32-node chunk): the Gram entries k_i.k_j and
//                           q_i.k_j of the chunk's nodes against their ancestors (MFMA over the 32 x 32 blocks
//                           below the diagonal), written per path slot: gram[node][key head][2][MAXD]. When the
//                           main kernel's grid fits on the CUs at once (one 257-node tree, HK 16 / H 32: 256
//                           workgroups), its workgroups compute the chunks themselves instead (one launch)
//   tree_gdn_large_kernel   one workgroup per (request, value head, 16 or 32 value columns), LDS sized by the
//                           largest tree of the call: path coefficients a and p, the rows of T = (I + A)^{-1} by
//                           path-local back substitution, R and E on MFMA (S0 rounded to bf16, as the reference),
//                           then u_i = sum_s T_i[s] R_path(i,s) and o_i = E_i + sum_s p_i[s] u_path(i,s) (fp32
//                           gathers along the root path: o takes u of the ancestors, so W = P T is never formed)
// The sub-units of one (request, key head) sit on one XCD, so its q / k rows and Gram rows are read from
// HBM once and from that XCD's L2 after.
#include <mutex>

#include "gdn_common.h"

namespace {
using namespace gdn;

// Tree context of one request for the large-tree path (global memory; one block per request).
template <int NMAX>
struct alignas(16) TreeMetaL {
  uint16_t path[NMAX][MAXD];  // path[i][s] = ancestor of i at depth s + 1 for s < depth[i] (path[i][depth-1] = i);
                              // i for s >= depth[i]; 0 for i >= n
  uint8_t depth[NMAX];        // nodes on the root path of i (0 for i >= n)
  int32_t bad;                // MFD_DEVERR_* bits of the tree
  int32_t n;                  // nodes of the request
  int32_t nmax;               // NMAX of the layout
  int32_t pad;
};
static_assert(sizeof(TreeMetaL<256>) % 16 == 0 && sizeof(TreeMetaL<512>) % 16 == 0, "16-byte copies");
template <int NMAX>
constexpr uint32_t meta_depth_off() { return (uint32_t)(NMAX * MAXD * 2); }

template <int NMAX>
__global__ __launch_bounds__(NMAX) void tree_ctx_large_kernel(const int32_t* parents, const int8_t* anc8,
                                                              const int32_t* cu_nodes, int N, uint8_t* ctx,
                                                              int32_t* err) {
  __shared__ TreeMetaL<NMAX> m;
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
  const int live = fits && tid < n;
  par[tid] = live ? parent_of(parents, anc8, ns, tid, n) : -1;
  __syncthreads();
  // walk up the parents; the chain stays in registers
  int d = 0;
  int chain[MAXD + 1];
  if (live) {
    int cur = tid;
#pragma unroll
    for (int s = 0; s <= MAXD; ++s) {
      chain[s] = cur;
      if (cur >= 0) {
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
      d = 0;
    }
  }
  const uint16_t self = (uint16_t)(live ? tid : 0);
#pragma unroll
  for (int s = 0; s < MAXD; ++s) m.path[tid][s] = self;
#pragma unroll
  for (int s = 0; s < MAXD; ++s)
    if (s < d) m.path[tid][d - 1 - s] = (uint16_t)chain[s];
  m.depth[tid] = (uint8_t)d;
  __syncthreads();
  if (tid == 0 && m.bad && err) atomicOr(err, m.bad);
  constexpr int NCM = (int)(sizeof(TreeMetaL<NMAX>) / 16);
  const uint4* src = reinterpret_cast<const uint4*>(&m);
  uint4* dst = reinterpret_cast<uint4*>(ctx + (size_t)r * sizeof(TreeMetaL<NMAX>));
  for (int c = tid; c < NCM; c += NMAX) dst[c] = src[c];
}

// Gram rows of 32 nodes (chunk T of request r) for key head hk: gram[node][hk] = {k_i.k_path(i,s) for s < MAXD,
// q_i.k_path(i,s) for s < MAXD} (0 past the depth; the k.k slot of i itself is 0). One workgroup of eight waves per
// (request x key head, chunk); workgroup id -> (p, T) with id mod 8 = p mod 8, so the chunks of one (request, key
// head) share an XCD and the K rows they all read come from its L2 after the first. Wave w takes the 32 x 32 blocks
// (T, J) for J = w and w + 8 (J <= T) on v_mfma_f32_32x32x16_bf16. Every global load (the chunk's root paths, its K /
// Q rows, staged once in LDS for all waves' A fragments, the K rows and depths of the wave's blocks) is issued before
// any is used; which entries lie on a root path comes from one bit mask per column node (bit row: node 32 J + j is on
// the root path of i0 + row), built by one LDS atomic per (row, path slot).
// Blocks jlo .. jhi only (a part of the chunk): entries whose ancestor lies in another block are left to the
// call that computes it, and the slots past the depth (zeros) to the part with jlo = 0.
template <int NMAX, bool LOWREG = false>
__device__ __forceinline__ void gram_chunk(const GdnLargeArgs& a, int hk, int T, int ns, int n,
                                           const TreeMetaL<NMAX>* m, float (*kq)[2 * MAXD], uint32_t (*onpath)[32],
                                           u32x4 (*kqa)[32 * 16], int jlo = 0, int jhi = -1) {
  if (jhi < 0) jhi = T;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i0 = 32 * T;
  const int g2 = lane >> 5, l32 = lane & 31;
  const int HKD = a.HK * D;
  // thread (row, slot): the path entry and the row's depth first (their loads are the first to be waited for)
  const int prow = tid >> 4, pslot = tid & 15;
  int pj = 0, pd = 0;
  if (i0 + prow < n) {
    pj = m->path[i0 + prow][pslot];
    pd = m->depth[i0 + prow];
  }
  // slot of the B rows of the wave's blocks (depth - 1; -1 past the request's end)
  int sjv[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int j = 32 * (w + 8 * x) + l32;
    sjv[x] = (w + 8 * x >= jlo && w + 8 * x <= jhi && j < n) ? (int)m->depth[j] - 1 : -1;
  }
  // the chunk's K and Q rows into LDS once (direct-to-LDS loads; chunk c of row r at 16-byte position
  // 16 r + (c ^ (r & 15)), so that the 32 rows of an A fragment read fall in different banks; rows past the request's
  // end repeat its last row), and the B fragments of the wave's blocks (rows 32 J + l32; past the end: zero)
  {
    const uint16_t* kb = a.k + ((size_t)ns * a.HK + hk) * D;
    const uint16_t* qb = a.q + ((size_t)ns * a.HK + hk) * D;
    // 1024 16-byte pieces (512 of K, 512 of Q), two instructions per wave
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int sl = (w * 2 + x) * 64 + lane;   // 0 .. 1023
      const int mat = sl >> 9, pos = sl & 511, rr = pos >> 4, cc = (pos & 15) ^ (rr & 15);
      const uint32_t off = (uint32_t)(min(i0 + rr, n - 1) * HKD + 8 * cc) * 2u;
      dma16_s(mat ? qb : kb, off, lds_addr(&kqa[0][0]) + (uint32_t)((w * 2 + x) * 64) * 16u);
    }
  }
  const __amdgpu_buffer_rsrc_t rs_k = rsrc(a.k + ((size_t)ns * a.HK + hk) * D, (uint32_t)n * HKD * 2);
  // (LOWREG: the second block's B rows, which only chunks past the eighth have, are loaded once the first block's
  // products are done, so that one block's fragments are live at a time)
  u32x4 fb[2][D / 16];
  auto load_b = [&](int x) __attribute__((always_inline)) {
    const uint32_t off = (uint32_t)((32 * (w + 8 * x) + l32) * HKD + 8 * g2) * 2u;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
      fb[x][ks] = (w + 8 * x >= jlo && w + 8 * x <= jhi)
                      ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_k, off + ks * 32, 0, 0))
                      : (u32x4){0u, 0u, 0u, 0u};
  };
  load_b(0);
  if constexpr (!LOWREG) load_b(1);
  reinterpret_cast<float*>(&kq[0][0])[tid] = 0.f;
  reinterpret_cast<float*>(&kq[0][0])[tid + 512] = 0.f;
  if (tid < NMAX) reinterpret_cast<uint32_t*>(&onpath[0][0])[tid] = 0u;
  wait_vmcnt<0>();  // the direct-to-LDS rows (and everything else) have landed
  __syncthreads();
  if (pslot < pd) atomicOr(&onpath[pj >> 5][pj & 31], 1u << prow);
  __syncthreads();
  // A fragments: lane row l32, k = 16 ks + 8 g2 .. + 7 (piece 2 ks + g2); held in registers for both blocks, or
  // (LOWREG) read again per block, next to their products
  u32x4 fa[D / 16], fq[D / 16];
  auto read_a = [&](int ks) __attribute__((always_inline)) {
    const int pos = 16 * l32 + ((2 * ks + g2) ^ (l32 & 15));
    fa[ks] = kqa[0][pos];
    fq[ks] = kqa[1][pos];
  };
  if constexpr (!LOWREG) {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) read_a(ks);
  }
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    if (w + 8 * x > jhi) break;
    if (w + 8 * x < jlo) continue;
    if constexpr (LOWREG) {
      if (x == 1) {
        load_b(1);
        wait_vmcnt<0>();
      }
    }
    const int J = w + 8 * x;
    const int j = 32 * J + l32;
    const uint32_t msk = onpath[J][l32];
    f32x16 gkk = {}, gqk = {};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      if constexpr (LOWREG) read_a(ks);
      gkk = mfma32(__builtin_bit_cast(bf16x8, fa[ks]), __builtin_bit_cast(bf16x8, fb[x][ks]), gkk);
      gqk = mfma32(__builtin_bit_cast(bf16x8, fq[ks]), __builtin_bit_cast(bf16x8, fb[x][ks]), gqk);
      if constexpr (LOWREG) __builtin_amdgcn_sched_barrier(0);  // keep the reads next to their products
    }
    // C register e: row 8 (e / 4) + 4 g2 + e % 4, column j, kept where j is on that row's root path (slot sjv)
    const int sj = sjv[x];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = 8 * (e >> 2) + 4 * g2 + (e & 3);
      if ((msk >> row) & 1u) {
        kq[row][MAXD + sj] = gqk[e];
        if (j != i0 + row) kq[row][sj] = gkk[e];
      }
    }
  }
  __syncthreads();
  if (jlo == 0 && jhi == T) {
    if (tid < 256) {
      const int row = tid >> 3, c = tid & 7;
      if (i0 + row < n) {
        float* gb = a.gram + (((size_t)ns + i0 + row) * a.HK + hk) * (2 * MAXD);
        *reinterpret_cast<f32x4*>(gb + 4 * c) = *reinterpret_cast<const f32x4*>(&kq[row][4 * c]);
      }
    }
  } else if (i0 + prow < n && (pslot < pd ? (pj >> 5) >= jlo && (pj >> 5) <= jhi : jlo == 0)) {
    // a part: thread (row, slot) stores the two entries of its slot that the part owns
    float* gb = a.gram + (((size_t)ns + i0 + prow) * a.HK + hk) * (2 * MAXD);
    gb[pslot] = kq[prow][pslot];
    gb[MAXD + pslot] = kq[prow][MAXD + pslot];
  }
}

// Gram work units of a request of nch chunks in the one-launch form, with sub_count workgroups in its group: the
// chunks, the largest of those with more than four blocks cut in two halves while the group has workgroups to spare
// (one 257-node tree, 16 workgroups: chunks 4-8 in halves, 14 units), so that no workgroup loads the B rows of
// more than about half a chunk's blocks. Unit vc < nch: chunk vc (its lower half when cut); unit nch + x: the
// upper half of chunk nch - 1 - x.
__device__ __forceinline__ int gram_nsplit(int nch, int sub_count) { return max(0, min(nch - 4, sub_count - nch)); }
__device__ __forceinline__ void gram_unit(int vc, int nch, int nsplit, int& T, int& jlo, int& jhi) {
  if (vc < nch) {
    T = vc;
    jlo = 0;
    jhi = T >= nch - nsplit ? (T + 1) / 2 - 1 : T;
  } else {
    T = nch - 1 - (vc - nch);
    jlo = (T + 1) / 2;
    jhi = T;
  }
}

// at most 128 VGPRs (four waves per SIMD): two workgroups per CU
template <int NMAX>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(6, 6))) void tree_gram_kernel(GdnLargeArgs a,
                                                                                                  int nchunks) {
  const int P = a.R * a.HK;
  const int P8 = (P + 7) >> 3;
  const int id = blockIdx.x;
  const int rest = id >> 3;
  const int pidx = (rest % P8) * 8 + (id & 7);
  // the chunks with the most blocks first, so that the workgroups that start last (past the first round of two per
  // CU) are the cheapest
  const int T = nchunks - 1 - rest / P8;
  if (pidx >= P || T < 0) return;
  const int r = pidx / a.HK;
  const int hk = pidx % a.HK;
  int ns, n;
  request_range(a.cu_nodes, r, a.N, ns, n);
  if (32 * T >= n || n > NMAX) return;
  const TreeMetaL<NMAX>* m = reinterpret_cast<const TreeMetaL<NMAX>*>(a.ctx) + r;
  if (m->bad != 0 || m->n != n || m->nmax != NMAX) return;  // rejected: the main kernel reports it

  __shared__ float kq[32][2 * MAXD];
  __shared__ uint32_t onpath[NMAX / 32][32];
  __shared__ u32x4 kqa[2][32 * 16];  // the chunk's K rows, then its Q rows (16-byte pieces, swizzled)
  gram_chunk<NMAX, true>(a, hk, T, ns, n, m, kq, onpath, kqa);
}

// Dynamic LDS of the main kernel for trees of at most nml nodes (nml a multiple of 16) and CT 16-column tiles (CW =
// 16 CT value columns); float strides padded by 4 (2 for S0) where the total allows it, so that the rows a wave
// reads or writes together fall in different banks:
//   kq   [nml][2 MAXD] f32   Gram row of node i (k.k slots, then q.k slots) -> a_i (strict ancestors), p_i
//   t    [nml][ts] f32       T_i[s] (0 past the depth); before phase T the S0 slice [D][ss] f32 (k rows of the CW
//                            value columns) lies here
//   ru   [nml][rs] f32       R rows of the workgroup's value columns, then u rows
//   path [nml][MAXD] u16, g [nml] f32, beta [nml] f32, depth [nml] i32
struct LargeLds {
  int ts, rs, ss;
  uint32_t kq, t, ru, path, g, beta, dep, total;
};
__host__ __device__ inline LargeLds large_lds(int nml, int ct) {
  LargeLds L{};
  const int cw = 16 * ct;
  for (int pad = 1; pad >= 0; --pad) {
    L.ts = MAXD + 4 * pad;
    L.rs = cw + 4 * pad;
    L.ss = cw + 2 * pad;
    L.kq = 0;
    L.t = L.kq + (uint32_t)nml * 2 * MAXD * 4;
    const uint32_t tbytes = (uint32_t)nml * L.ts * 4, sbytes = (uint32_t)D * L.ss * 4;
    L.ru = L.t + (tbytes > sbytes ? tbytes : sbytes);
    L.path = L.ru + (uint32_t)nml * L.rs * 4;
    L.g = L.path + (uint32_t)nml * MAXD * 2;
    L.beta = L.g + (uint32_t)nml * 4;
    L.dep = L.beta + (uint32_t)nml * 4;
    L.total = L.dep + (uint32_t)nml * 4;
    if (L.total <= 160u * 1024u) break;
  }
  return L;
}
// Hand-over words of the one-launch form, per (request, key head) group: [0] the group's call count, [1] its
// workgroups done with this call's Gram rows, [2 + c] the tag of Gram unit c once it is written (call count + 1,
// and the writer's XCD). A library array (512 KiB), zero at load, in GSYNC_SLOTS sets: each stream that runs the
// form gets a set of its own (calls on one stream never overlap, so they can share one). The form engages only when
// the whole grid fits on the CUs, i.e. for at most 256 / 5 groups on MI355X.
constexpr int GSYNC_GROUPS = 64;
constexpr int GSYNC_WORDS = 32;
constexpr int GSYNC_SLOTS = 64;
__device__ __align__(256) uint32_t gsync_words[GSYNC_SLOTS * GSYNC_GROUPS * GSYNC_WORDS];
// scratch offsets of a Gram chunk inside the main kernel's LDS (from the KQ region on)
constexpr uint32_t GRAM_SCR_ONPATH = 32 * 2 * MAXD * 4;                    // after kq [32][2 MAXD] f32
constexpr uint32_t GRAM_SCR_KQA = GRAM_SCR_ONPATH + 512 / 32 * 32 * 4;     // after onpath [NMAX / 32][32] u32
constexpr uint32_t GRAM_SCR_MISS = GRAM_SCR_KQA + 2 * 32 * 16 * 16;        // after kqa [2][512] 16-byte pieces
constexpr uint32_t GRAM_SCR_BYTES = GRAM_SCR_MISS + 16;

// The Gram rows of request (ns, n) and key head hk (8 pieces of 16 bytes per node) into LDS at KQ (direct loads)
__device__ __forceinline__ void gram_rows_to_lds(const GdnLargeArgs& a, int ns, int hk, int ngr, float* KQ, int w,
                                                 int lane) {
  const float* gb = a.gram + ((size_t)ns * a.HK + hk) * (2 * MAXD);
  for (int cc = w * 64; cc < ngr; cc += 512) {
    const int c = cc + lane;
    if (c < ngr)
      dma16_s(gb, (uint32_t)((c >> 3) * a.HK * (2 * MAXD) + (c & 7) * 4) * 4u, lds_addr(KQ) + (uint32_t)cc * 16u);
  }
}

constexpr int LT = 512;  // threads of the main kernel: one per node in phase T
constexpr int PRE = 2;   // 16-node tiles whose K / Q rows and v are requested before phase T

// One workgroup per (request, value head, CW = 16 CT value columns), eight waves; wave w owns the 16-node tiles
// t = w, w + 8, ... of the R, U and O phases, for all CT 16-column tiles.
//   0  root paths and Gram rows straight into LDS, depths and gates, the S0 slice (LDS, padded rows) (one-launch
//      form: workgroup sub computes Gram units sub, sub + SUB, ... (chunks or halves of chunks) while these loads
//      are in flight and publishes them; the Gram rows are loaded once every unit of the group is published, after
//      the S0 fragments); then each wave's S0 B fragments (bf16, rounded as the reference's s_blk); after phase A
//      the first PRE tiles' K / Q rows (A fragments) and v are requested, in flight through phase T (requested with
//      phase 0's loads, they waited behind them at issue)
//   A  (eight threads per node, one per four slots) a_i[s] = beta_i e^{G_i - G_j} k_i.k_j (s < depth - 1),
//      p_i[s] = e^{G_i - G_j} q_i.k_j (s < depth)
//   T  (one thread per node) the row of T = (I + A)^{-1} on i's root path, by right-looking back substitution
//   R  per 16-node tile and 16-column tile on MFMA: K S0 and Q S0; a quad transpose gives each lane one node and four
//      consecutive columns: R = beta (v - e^G K S0) into LDS, E = e^G Q S0 in registers (the tile after next
//      requested); waves without a T job start here at once
//   U  u_i = sum_{s < depth} T_i[s] R_path(i,s) (16-byte gathers; registers, then over R in LDS)
//   O  o_i = E_i + sum_{s < depth} p_i[s] u_path(i,s); u and o leave as 16-byte stores
// ONE: the one-launch form (a.gsync set); a separate instantiation, so that the two-kernel form keeps its registers
template <int NMAX, int CT, bool ONE>
__global__ __launch_bounds__(LT) void tree_gdn_large_kernel(GdnLargeArgs a, int nml) {
  constexpr int CW = 16 * CT;                 // value columns of a workgroup
  constexpr int MAXT = (NMAX / 16 + 7) / 8;   // 16-node tiles per wave at most
  extern __shared__ __align__(16) uint8_t lds[];
  const LargeLds L = large_lds(nml, CT);
  const int TS = L.ts, RS = L.rs, SS = L.ss;
  float* const KQ = reinterpret_cast<float*>(lds + L.kq);
  float* const TT = reinterpret_cast<float*>(lds + L.t);
  float* const S0L = reinterpret_cast<float*>(lds + L.t);
  float* const RU = reinterpret_cast<float*>(lds + L.ru);
  uint16_t* const PT = reinterpret_cast<uint16_t*>(lds + L.path);
  float* const Gs = reinterpret_cast<float*>(lds + L.g);
  float* const Bs = reinterpret_cast<float*>(lds + L.beta);
  int* const DP = reinterpret_cast<int*>(lds + L.dep);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4;
  const int l16 = lane & 15;

  // workgroup -> (request, key head, value head member x column group); the sub-units of one (request, key head)
  // land on one XCD (workgroup id modulo 8), so its q / k rows and Gram rows come from that XCD's L2 after the first
  const int Gq = a.H / a.HK;
  const int NCGW = D / CW;
  const int SUB = Gq * NCGW;
  const int P = a.R * a.HK;
  const int id = blockIdx.x;
  const int rest = id >> 3;
  const int pidx = (rest / SUB) * 8 + (id & 7);
  if (pidx >= P) return;
  const int sub = rest % SUB;
  const int r = pidx / a.HK;
  const int hk = pidx % a.HK;
  const int h = hk * Gq + sub / NCGW;
  const int cg = sub % NCGW;
  int ns, n;
  request_range(a.cu_nodes, r, a.N, ns, n);
  ns = __builtin_amdgcn_readfirstlane(ns);
  n = __builtin_amdgcn_readfirstlane(n);
  if (n <= 0) return;
  const TreeMetaL<NMAX>* m = reinterpret_cast<const TreeMetaL<NMAX>*>(a.ctx) + r;
  const int rej = (n > NMAX || n > nml)
                      ? MFD_DEVERR_TOO_MANY_NODES
                      : (m->bad | ((m->n != n || m->nmax != NMAX) ? MFD_DEVERR_BAD_CONTEXT : 0));
  if (rej) {
    nan_fill(a.u, a.o, ns, n, a.H, h, cg * CW, CW, tid, LT);
    if (tid == 0 && a.err) atomicOr(a.err, rej);
    return;
  }
  const int HD = a.H * D, HKD = a.HK * D;
  const int nt16 = (n + 15) >> 4;
  const int cb = cg * CW;  // first value column of the workgroup
  // one-launch form: the request's Gram chunks are computed by the first nch workgroups of its (request, key head)
  // group (sub = chunk) and handed over through global memory (below); gen = the group's call count, read before
  // anything of this call is published
  constexpr bool fused = ONE;
  const int nch = (n + 31) >> 5;
  const int nsplit = gram_nsplit(nch, SUB);
  const int nvc = nch + nsplit;  // Gram work units of the group
  uint32_t* const gsy = fused ? a.gsync + (size_t)pidx * GSYNC_WORDS : nullptr;
  const uint32_t gen = fused ? (uint32_t)__builtin_amdgcn_readfirstlane(
                                   (int)__hip_atomic_load(gsy, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                             : 0u;
  // a chunk word: this call's count + 1 in bits 31..4, the writer's XCD in bits 3..0
  uint32_t xcc = 0;
  if (fused) asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
  const uint32_t tag = ((gen + 1u) << 4) | xcc;
  // a Gram chunk's scratch (kq 4 KB, onpath 2 KB, kqa 16 KB, then a word of missing-chunk bits): the KQ region and
  // on, free until the group's Gram rows are loaded; it ends before the root paths, gates and depths
  uint8_t* const scr = lds + L.kq;
  float (*const gkq)[2 * MAXD] = reinterpret_cast<float (*)[2 * MAXD]>(scr);
  uint32_t (*const gon)[32] = reinterpret_cast<uint32_t (*)[32]>(scr + GRAM_SCR_ONPATH);
  u32x4 (*const gkqa)[32 * 16] = reinterpret_cast<u32x4 (*)[32 * 16]>(scr + GRAM_SCR_KQA);
  uint32_t* const gmiss = reinterpret_cast<uint32_t*>(scr + GRAM_SCR_MISS);

  // ---- phase 0
  {
    const int np = 2 * n, ngr = 8 * n;
    for (int cc = w * 64; cc < np; cc += LT)
      if (cc + lane < np) dma16_s(m, (uint32_t)(cc + lane) * 16u, lds_addr(PT) + (uint32_t)cc * 16u);
    if (!fused) gram_rows_to_lds(a, ns, hk, ngr, KQ, w, lane);
    // the S0 slice: D rows of CW columns, CT 16-byte pieces per thread (thread x: row x / (CW / 4), piece x % (CW / 4))
    const float* s0b = a.s0 + ((size_t)r * a.H + h) * D * D + cb;
    u32x4 s0p[CT];
#pragma unroll
    for (int x = 0; x < CT; ++x) {
      const int c = tid + LT * x;
      s0p[x] = *reinterpret_cast<const u32x4*>(s0b + (size_t)(c / (CW / 4)) * D + 4 * (c % (CW / 4)));
    }
    float g = 0.f, b = 0.f;
    int d = 0;
    if (tid < n) {
      g = a.g_cum[(size_t)(ns + tid) * a.H + h];
      b = a.beta[(size_t)(ns + tid) * a.H + h];
      d = m->depth[tid];
    }
    // this workgroup's Gram units (sub, sub + SUB, ...) while the loads above are in flight; publish: a unit's
    // stores have completed (in this XCD's L2, which every workgroup of the group shares), then its word takes this
    // call's tag. The barrier also ends the unit's use of the scratch (the next unit's, or the S0 slice's)
    for (int vc = fused ? sub : nvc; vc < nvc; vc += SUB) {
      int T, jlo, jhi;
      gram_unit(vc, nch, nsplit, T, jlo, jhi);
      gram_chunk<NMAX>(a, hk, T, ns, n, m, gkq, gon, gkqa, jlo, jhi);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) __hip_atomic_store(gsy + 2 + vc, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_vmcnt<0>();
    if (tid < nml) {
      Gs[tid] = g;
      Bs[tid] = b;
      DP[tid] = d;
    }
#pragma unroll
    for (int x = 0; x < CT; ++x) {
      const int c = tid + LT * x;
      float* dst = S0L + (c / (CW / 4)) * SS + 4 * (c % (CW / 4));
      *reinterpret_cast<u32x2*>(dst) = (u32x2){s0p[x][0], s0p[x][1]};
      *reinterpret_cast<u32x2*>(dst + 2) = (u32x2){s0p[x][2], s0p[x][3]};
    }
  }
  // K / Q rows of a tile as A fragments (lane: node 16 t + l16, dims 32 kc + 8 g4 .. + 7) and v of its nodes in the
  // transposed layout (lane: node 16 t + 4 g4 + (l16 & 3), columns cb + 16 ct + 4 (l16 >> 2) .. + 3); rows past the
  // request's end read as zero
  const __amdgpu_buffer_rsrc_t rs_k = rsrc(a.k + ((size_t)ns * a.HK + hk) * D, (uint32_t)n * HKD * 2);
  const __amdgpu_buffer_rsrc_t rs_q = rsrc(a.q + ((size_t)ns * a.HK + hk) * D, (uint32_t)n * HKD * 2);
  const __amdgpu_buffer_rsrc_t rs_v = rsrc(a.v + ((size_t)ns * a.H + h) * D, (uint32_t)n * HD * 2);
  const int tn = 4 * g4 + (l16 & 3);      // node of this lane within a tile (transposed layout)
  const int tc = 4 * (l16 >> 2);          // first of this lane's four columns within a 16-column tile
  u32x4 fk[2][D / 32], fq[2][D / 32];
  u32x2 vv[2][CT];
  auto load_tile = [&](int t, int slot) __attribute__((always_inline)) {
    const uint32_t off = (uint32_t)((16 * t + l16) * HKD + 8 * g4) * 2u;
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc) {
      fk[slot][kc] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_k, off + kc * 64, 0, 0));
      fq[slot][kc] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_q, off + kc * 64, 0, 0));
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
      vv[slot][ct] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
          rs_v, (uint32_t)((16 * t + tn) * HD + cb + 16 * ct + tc) * 2u, 0, 0));
  };
  __syncthreads();
  // S0 B fragments of this wave's column tiles: column cb + 16 ct + l16, k = 32 kc + 8 g4 .. + 7
  bf16x8 sb[CT][D / 32];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc) {
      const float* src = S0L + (32 * kc + 8 * g4) * SS + 16 * ct + l16;
      u32x4 pk;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pk[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){src[(2 * e) * SS], src[(2 * e + 1) * SS]}, bf16x2));
      sb[ct][kc] = __builtin_bit_cast(bf16x8, pk);
    }

  if (fused) {
    __syncthreads();  // every wave has its S0 fragments: the T region is free again (scratch of a local chunk)
    // wait for the group's Gram units (bounded); a unit that has not come, or that was written on another XCD (whose
    // L2 this one does not see), is computed here as well (the same entries, so the producer's writes carry the same
    // values): never a hang, never a stale row
    bool missing = false;
    if (tid < nvc) {
      missing = true;
      for (int it = 0; it < (1 << 16); ++it) {
        const uint32_t v = __hip_atomic_load(gsy + 2 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((v >> 4) == (tag >> 4)) {
          missing = v != tag;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    if (w == 0) {
      const uint64_t mb = __builtin_amdgcn_ballot_w64(missing);
      if (lane == 0) *gmiss = (uint32_t)mb;
    }
    __syncthreads();
    const uint32_t miss = *gmiss;
    if (miss != 0u) {
      for (int vc = 0; vc < nvc; ++vc)
        if ((miss >> vc) & 1u) {
          __syncthreads();  // the scratch of the previous unit is free
          int T, jlo, jhi;
          gram_unit(vc, nch, nsplit, T, jlo, jhi);
          gram_chunk<NMAX, true>(a, hk, T, ns, n, m, gkq, gon, gkqa, jlo, jhi);  // (rare: fewer registers)
        }
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();  // scratch dead; every row of the group is in memory
    gram_rows_to_lds(a, ns, hk, 8 * n, KQ, w, lane);
    wait_vmcnt<0>();
    __syncthreads();
    // this workgroup is done with the group's rows: the last of the group's SUB workgroups starts the next call's
    // count (every workgroup of the group read gen before counting itself here)
    if (tid == 0) {
      const uint32_t old = __hip_atomic_fetch_add(gsy + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old == (uint32_t)SUB - 1u) {
        __hip_atomic_store(gsy + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(gsy, gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }

  // ---- phase A: a_i (strict ancestors, slots 0-15) and p_i (slots 16-31) in place; thread x: node x / 8, slots
  //      4 (x % 4) .. + 3 of part (x / 4) % 2
  for (int x = tid; x < 8 * n; x += LT) {
    const int i = x >> 3, c = x & 7, s4 = 4 * (c & 3);
    const bool pp_part = (c & 4) != 0;
    const float gi = Gs[i];
    const float sc = pp_part ? 1.f : Bs[i];
    const int d = DP[i];
    const int lim = pp_part ? d : d - 1;
    f32x4 xv = *reinterpret_cast<const f32x4*>(&KQ[i * 2 * MAXD + 4 * c]);
    const u32x2 pp = *reinterpret_cast<const u32x2*>(&PT[i * MAXD + s4]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = (int)((pp[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      const float ex = __expf(gi - Gs[s4 + e < d ? j : i]);
      xv[e] = (s4 + e < lim) ? xv[e] * (sc * ex) : 0.f;
    }
    *reinterpret_cast<f32x4*>(&KQ[i * 2 * MAXD + 4 * c]) = xv;
  }
  // the first tiles' K / Q rows and v, in flight during T: waves 0-3 (the T threads of the first 256 nodes) request
  // theirs before the barrier, the others after it, where their issue (a wave waits there for room in the CU's
  // load queue) runs beside T instead of holding the barrier
  if (w < 4) {
#pragma unroll
    for (int j = 0; j < PRE; ++j) load_tile(w + 8 * j, j);
  }
  __syncthreads();  // coefficients complete; the S0 slice is dead (phase T writes over it)
  if (w >= 4) {
#pragma unroll
    for (int j = 0; j < PRE; ++j) load_tile(w + 8 * j, j);
  }

  // ---- phase T: T_i[d-1] = 1, T_i[s] = -sum_{m>s} T_i[m] a_{path(m)}[s] (right-looking over m)
  if (tid < n) {
    const int i = tid;
    const int d = DP[i];
    int pth[MAXD];
#pragma unroll
    for (int s4 = 0; s4 < MAXD; s4 += 4) {
      const u32x2 pp = *reinterpret_cast<const u32x2*>(&PT[i * MAXD + s4]);
#pragma unroll
      for (int e = 0; e < 4; ++e) pth[s4 + e] = (int)((pp[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
    }
    float acc[MAXD], Tr[MAXD];
#pragma unroll
    for (int s = 0; s < MAXD; ++s) acc[s] = 0.f;
#pragma unroll
    for (int mm = MAXD - 1; mm >= 0; --mm) {
      const float tm = (mm < d) ? ((mm == d - 1) ? 1.f : -acc[mm]) : 0.f;
      Tr[mm] = tm;
      if (mm > 0 && mm < d) {
        const float* row = &KQ[pth[mm] * 2 * MAXD];
#pragma unroll
        for (int s4 = 0; s4 < mm; s4 += 4) {
          const f32x4 rv = *reinterpret_cast<const f32x4*>(row + s4);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (s4 + e < mm) acc[s4 + e] = fmaf(tm, rv[e], acc[s4 + e]);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < MAXD; s += 4)
      *reinterpret_cast<f32x4*>(&TT[i * TS + s]) = (f32x4){Tr[s], Tr[s + 1], Tr[s + 2], Tr[s + 3]};
  }

  // ---- phase R (no barrier before it: R writes only the ru region and reads the gates)
  f32x4 E[MAXT][CT];
#pragma unroll
  for (int j = 0; j < MAXT; ++j) {
    const int t = w + 8 * j;
    if (t >= nt16) break;
    const int slot = j & 1;
    const int i = 16 * t + tn;
    const float eg = __expf(Gs[i]);
    const float bi = Bs[i];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      f32x4 ak = {0.f, 0.f, 0.f, 0.f}, aq = ak;
#pragma unroll
      for (int kc = 0; kc < D / 32; ++kc) {
        ak = mfma16(__builtin_bit_cast(bf16x8, fk[slot][kc]), sb[ct][kc], ak);
        aq = mfma16(__builtin_bit_cast(bf16x8, fq[slot][kc]), sb[ct][kc], aq);
      }
      // C layout (column 16 ct + l16, nodes 4 g4 .. + 3) -> node tn, columns tc .. tc + 3
      const f32x4 kt = quad_transpose(ak, lane);
      const f32x4 qt = quad_transpose(aq, lane);
      const u32x2 vb = vv[slot][ct];
      const f32x4 vf = {bf2f((uint16_t)(vb[0] & 0xFFFFu)), bf2f((uint16_t)(vb[0] >> 16)), bf2f((uint16_t)(vb[1] & 0xFFFFu)),
                        bf2f((uint16_t)(vb[1] >> 16))};
      f32x4 rv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        rv[e] = bi * (vf[e] - eg * kt[e]);
        E[j][ct][e] = eg * qt[e];
      }
      *reinterpret_cast<f32x4*>(&RU[i * RS + 16 * ct + tc]) = rv;
    }
    if (j + 2 < MAXT && t + 16 < nt16) load_tile(t + 16, slot);
  }
  __syncthreads();  // T rows and R rows complete

  // ---- phase U: u_i = sum_{s < depth} T_i[s] R_path(i,s) (lanes past the depth read row 0 with weight 0: one
  //      broadcast address instead of a row of their own)
  f32x4 U[MAXT][CT];
#pragma unroll
  for (int j = 0; j < MAXT; ++j) {
    const int t = w + 8 * j;
    if (t >= nt16) break;
    const int i = 16 * t + tn;
    const int d = DP[i];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) U[j][ct] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int s4 = 0; s4 < MAXD; s4 += 4) {
      if (__builtin_amdgcn_ballot_w64(s4 < d) == 0) break;
      const u32x2 pp = *reinterpret_cast<const u32x2*>(&PT[i * MAXD + s4]);
      const f32x4 tv = *reinterpret_cast<const f32x4*>(&TT[i * TS + s4]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bool on = s4 + q < d;
        const int jn = on ? (int)((pp[q >> 1] >> (16 * (q & 1))) & 0xFFFFu) : 0;
        const float wt = on ? tv[q] : 0.f;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const f32x4 rv = *reinterpret_cast<const f32x4*>(&RU[jn * RS + 16 * ct + tc]);
#pragma unroll
          for (int e = 0; e < 4; ++e) U[j][ct][e] = fmaf(wt, rv[e], U[j][ct][e]);
        }
      }
    }
  }
  __syncthreads();  // every R gather done
#pragma unroll
  for (int j = 0; j < MAXT; ++j) {
    const int t = w + 8 * j;
    if (t >= nt16) break;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) *reinterpret_cast<f32x4*>(&RU[(16 * t + tn) * RS + 16 * ct + tc]) = U[j][ct];
  }
  __syncthreads();  // u rows complete

  // ---- phase O: o_i = E_i + sum_{s < depth} p_i[s] u_path(i,s); u and o stored (16 bytes per lane and column tile)
  const __amdgpu_buffer_rsrc_t rs_u = rsrc(a.u + ((size_t)ns * a.H + h) * D, (uint32_t)n * HD * 4);
  const __amdgpu_buffer_rsrc_t rs_o = rsrc(a.o + ((size_t)ns * a.H + h) * D, (uint32_t)n * HD * 4);
#pragma unroll
  for (int j = 0; j < MAXT; ++j) {
    const int t = w + 8 * j;
    if (t >= nt16) break;
    const int i = 16 * t + tn;
    const int d = DP[i];
    for (int s4 = 0; s4 < MAXD; s4 += 4) {
      if (__builtin_amdgcn_ballot_w64(s4 < d) == 0) break;
      const u32x2 pp = *reinterpret_cast<const u32x2*>(&PT[i * MAXD + s4]);
      const f32x4 pv = *reinterpret_cast<const f32x4*>(&KQ[i * 2 * MAXD + MAXD + s4]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bool on = s4 + q < d;
        const int jn = on ? (int)((pp[q >> 1] >> (16 * (q & 1))) & 0xFFFFu) : 0;
        const float wt = on ? pv[q] : 0.f;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const f32x4 uv = *reinterpret_cast<const f32x4*>(&RU[jn * RS + 16 * ct + tc]);
#pragma unroll
          for (int e = 0; e < 4; ++e) E[j][ct][e] = fmaf(wt, uv[e], E[j][ct][e]);
        }
      }
    }
    const uint32_t off = (uint32_t)(i * HD + cb + tc) * 4u;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      store4(rs_u, off + 64 * ct, U[j][ct][0], U[j][ct][1], U[j][ct][2], U[j][ct][3]);
      store4(rs_o, off + 64 * ct, E[j][ct][0], E[j][ct][1], E[j][ct][2], E[j][ct][3]);
    }
  }
}

template <int NMAX, int CT, bool ONE>
int run_large_ct(const GdnLargeArgs& a, int nml, hipStream_t s) {
  const int lds = (int)large_lds(nml, CT).total;
  if (int rc = mfd_set_max_lds(reinterpret_cast<const void*>(&tree_gdn_large_kernel<NMAX, CT, ONE>), 160 * 1024))
    return rc;
  const int P = a.R * a.HK;
  const int SUB = (a.H / a.HK) * (D / (16 * CT));
  const dim3 grid(8 * ((P + 7) / 8) * SUB);
  hipLaunchKernelGGL((tree_gdn_large_kernel<NMAX, CT, ONE>), grid, dim3(LT), lds, s, a, nml);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

constexpr int MAX_DEVICES = 64;
struct GsyncDevice {
  uint32_t* base = nullptr;           // device address of this device's `gsync_words`, looked up once
  hipStream_t owner[GSYNC_SLOTS] = {};  // the stream each set belongs to
  int used = 0;
};
std::mutex g_gsync_mu;
GsyncDevice g_gsync[MAX_DEVICES];

// The hand-over set of stream s on the current device (the caller's stream belongs to it); null when every set is
// taken by other streams (the call then takes the two-kernel form).
int stream_gsync(hipStream_t s, uint32_t** out) {
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mfd_set_hip_error(e);
  if (dev < 0 || dev >= MAX_DEVICES) return MFD_OK;
  std::lock_guard<std::mutex> lock(g_gsync_mu);
  GsyncDevice& g = g_gsync[dev];
  if (!g.base) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(gsync_words));
    if (e != hipSuccess) return mfd_set_hip_error(e);
    g.base = static_cast<uint32_t*>(p);
  }
  int slot = 0;
  while (slot < g.used && g.owner[slot] != s) ++slot;
  if (slot == g.used) {
    if (g.used == GSYNC_SLOTS) return MFD_OK;
    g.owner[g.used++] = s;
  }
  *out = g.base + (size_t)slot * GSYNC_GROUPS * GSYNC_WORDS;
  return MFD_OK;
}

template <int NMAX>
int run_large(const GdnLargeArgs& a, int max_nodes, hipStream_t s) {
  const int nchunks = (max_nodes + 31) / 32;
  const int P = a.R * a.HK;
  const int P8 = (P + 7) / 8;
  const int nml = (max_nodes + 15) & ~15;
  // 32 value columns per workgroup while that still gives every CU a workgroup (the tree part is then shared by twice
  // the columns) and the LDS allows it; 16 otherwise
  const int cus = mfd_num_cus();
  const bool wide = (int64_t)a.R * a.H * (D / 32) >= cus && large_lds(nml, 2).total <= 160u * 1024u;
  const int ct = wide ? 2 : 1;
  const int SUB = (a.H / a.HK) * (D / (16 * ct));
  const LargeLds L = large_lds(nml, ct);
  // one launch when the whole grid fits on the CUs at once and each (request, key head) group has a workgroup per
  // Gram chunk: the chunks are then computed inside the main kernel while its phase-0 loads are in flight, instead
  // of by a kernel of their own before it. (With more workgroups than CUs the form still works, a workgroup taking
  // units sub, sub + SUB, ..., but a chunk costs about as long inside the main kernel as in its own kernel, and each
  // round of workgroups would pay for it: 4 x 257 nodes, 47.8 against 46.2 us.)
  GdnLargeArgs b = a;
  b.gsync = nullptr;
  if ((int64_t)8 * P8 * SUB <= cus && nchunks <= SUB && nchunks <= GSYNC_WORDS - 2 && P <= GSYNC_GROUPS &&
      L.path - L.kq >= GRAM_SCR_BYTES)
    if (int rc = stream_gsync(s, &b.gsync)) return rc;
  if (!b.gsync) {
    hipLaunchKernelGGL(tree_gram_kernel<NMAX>, dim3(8 * P8 * nchunks), dim3(512), 0, s, b, nchunks);
    MFD_CHECK_LAUNCH();
  }
  if (b.gsync) return wide ? run_large_ct<NMAX, 2, true>(b, nml, s) : run_large_ct<NMAX, 1, true>(b, nml, s);
  return wide ? run_large_ct<NMAX, 2, false>(b, nml, s) : run_large_ct<NMAX, 1, false>(b, nml, s);
}

}  // namespace

size_t gdn_large_ctx_block_bytes(int max_nodes) {
  return max_nodes <= 256 ? sizeof(TreeMetaL<256>) : sizeof(TreeMetaL<512>);
}

int gdn_large_context(const int32_t* parents, const int8_t* anc8, const int32_t* cu_nodes, int R, int N,
                      int max_nodes, uint8_t* ctx, int32_t* err, hipStream_t s) {
  if (max_nodes <= 256)
    hipLaunchKernelGGL(tree_ctx_large_kernel<256>, dim3(R), dim3(256), 0, s, parents, anc8, cu_nodes, N, ctx, err);
  else
    hipLaunchKernelGGL(tree_ctx_large_kernel<512>, dim3(R), dim3(512), 0, s, parents, anc8, cu_nodes, N, ctx, err);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}

int gdn_large_run(const GdnLargeArgs& a, int max_nodes, hipStream_t s) {
  return max_nodes <= 256 ? run_large<256>(a, max_nodes, s) : run_large<512>(a, max_nodes, s);
}
