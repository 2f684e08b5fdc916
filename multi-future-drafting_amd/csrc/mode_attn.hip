// K-mode drafter attention ("mode attention") for gfx950.
//
// Semantics (inference/hf/mode_attention.py:153-164 reference(); inference/sglang/patches/
// sglang-v0.5.22-mfd.patch:965-988): the K mode blocks of a request sit side by side (K x bs queries,
// mode-major). Query row (head h, query qi) of mode qi / bs attends to every context key of its request
// plus the bs block keys of its own mode (bidirectional inside the block unless causal_in_block);
// query head h reads KV head h / (H / Hkv). Softmax in base 2 with scale * log2(e), fp32 statistics.
//
// Work split: a workgroup takes one (request, KV head, context split, group of NW units); a unit is 32
// consecutive queries of one query head and runs on one wave (when K x bs is not a multiple of 32, the
// last unit of a head is padded with rows that compute a copy of its last query and store nothing). Workgroups are ordered longest request
// first, and the unit groups that share a (request, KV head, split) are consecutive on one XCD.
// NW = 4: two workgroups share a CU (two waves per SIMD: one wave alone cannot keep the MFMA pipe full);
// NW = 8 when a KV head's units come in eights: one workgroup per CU, each K / V tile loaded once per CU.
//
// The NW waves of a workgroup share 64-key K / V tiles that land in LDS straight from global memory
// (global_load_lds_dwordx4) in a ring of three K slots and two V slots (80 KB): K of tile t + 3 and V of
// tile t + 2 are loaded while tile t is processed. A tile is stored as [key][d] rows with an XOR swizzle
// of the 16-byte chunks so that both read patterns below are free of bank conflicts. Each wave computes
//   S^T = K Q^T   (v_mfma_f32_32x32x16_bf16: A = K rows from LDS, B = Q^T held in registers)
// so a lane owns one query row and the online-softmax state is a per-lane scalar, then
//   O^T += V^T P^T (A = V^T fragments read with ds_read_b64_tr_b16, the LDS transpose read, from the
//                   [key][d] tile; B = P^T straight from the S^T accumulators: the k order of a 16-key
//                   chunk is the C-register row order, so no data movement). This product runs in fp16
//                   (v_mfma_f32_32x32x16_f16): P rounded to fp16 (2^-12 relative; the reference rounds it
//                   to bf16, 2^-9, which with near-uniform attention costs about 1e-3 of the heavily
//                   cancelling average), V widened from bf16 to fp16 in place in LDS once per tile,
//                   each wave widening the quarter its own direct loads filled (exact for |v| in
//                   [2^-14, 65504]). A V value of magnitude 65536 or more becomes an infinity there, which
//                   leaves a non-finite accumulator in every column it touches; a workgroup that ends with
//                   one computes its tiles again one at a time with this product in bf16 (V as loaded, P
//                   as bf16 hi + lo), so such values cost time, not results.
// Within a wave, the scores of tile t + 1 (MFMA) are interleaved with the exponentials and the P V product
// of tile t in a fixed order of 32 MFMA slots, each slot's LDS operand read two slots ahead.
// The running max is rescaled lazily (only when a score exceeds it by more than 2^8), and only the last
// context tile and the block tiles are masked.
// The request's block keys are extra 64-key tiles with the mode mask: after the context in a single pass,
// or as a partial of their own when the context is split. One pass: the normalised output is written as
// bf16. Split: partials (O / l in fp16 with a power-of-two row scale, and lse) go to the workspace and a merge
// kernel combines them
// (inference/hf/mode_attention.py:91-117).
// Context keys come from a flat layout (slot = position), a page table whose power-of-two page size is
// at least 64 (a tile lies in one page: one table read per tile), or any per-key slot table (page
// size 1 = req_to_token, or other page sizes: slot = table[t / P] * P + t % P). Context lengths and
// table rows are read on the device, so the launch is graph safe.
#include "mfd_common.h"

namespace {

constexpr int D = 128;
constexpr int TK = 64;          // keys per tile
constexpr int TILE = TK * D;    // elements of one K or V tile (16 KB)
constexpr int NWAVES = 4;              // waves of a workgroup (units of 32 queries), or 8 (see the launch)
constexpr int UROWS = 32;       // queries per unit (one wave)
constexpr int KSLOTS = 3, VSLOTS = 2;

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// K slots 0..2 then V slots 0..1 (80 KB).
// Layout of a tile: 16-byte chunk c (d = 8c .. 8c + 7) of key r sits at chunk position
//   K: r * 16 + (c ^ (r & 15))        V: r * 16 + (c ^ ((r & 3) << 2))
__shared__ __attribute__((aligned(1024))) uint16_t lds_kv[(KSLOTS + VSLOTS) * TILE];

// One direct-to-LDS load (global_load_lds_dwordx4): lane l's 16 bytes land at LDS byte address
// lds_byte + 16 l (lds_byte is wave-uniform). Issued as inline asm so that the compiler's wait
// insertion does not treat every later LDS read as dependent on it: the kernel orders the ring itself
// (s_waitcnt vmcnt + s_barrier before a slot is read, s_barrier before it is refilled).
// Form 1: per-lane 64-bit address. Form 2: wave-uniform base + per-lane 32-bit byte offset.
// (Wave-uniform operands go through readfirstlane, which keeps them in SGPRs.)
__device__ __forceinline__ void dma16(const uint16_t* g, uint32_t lds_byte) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds_byte);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(l), "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void dma16_s(const uint16_t* base, uint32_t off, uint32_t lds_byte) {
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
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Workgroup barrier that is also a compiler memory barrier: LDS reads of a ring slot may not be moved
// across it (the s_barrier builtin alone does not order memory operations for the compiler).
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

struct AttnArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kn;
  const uint16_t* vn;
  int kn_st, vn_st;        // row strides (elements) of the block keys / values: < 2^31 / (K * L)
  int64_t kn_sh, vn_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int kc_ss, vc_ss;        // slot strides (elements) of the caches: < 2^31, slot ids are int32
  int64_t kc_sh, vc_sh;
  const int32_t* table;
  int64_t table_stride;
  int page_size;
  int page_shift;  // log2(page_size) when page_size is a power of two, else -1
  const int64_t* req_idx;
  const int64_t* ctx_lens;
  int ctx_const;
  uint16_t* out;
  int64_t o_st, o_sh;
  uint16_t* ws_o;  // [S][bs * H * KL][D] fp16: the partial output row divided by 2^ws_exp
  float* ws_lse;   // [S][bs * H * KL]
  float* ws_exp;   // [S][bs * H * KL] the row's power-of-two scale exponent
  int bs, K, L, H, Hkv, G, S, SC, causal;  // S partials per (request, KV head): SC context splits + 1 block
  float scale_log2;
  int ngroups;    // unit groups (of NW units, the kernel's waves) per (request, KV head)
};

// Combine a value with the one in the other 32-lane half of the wave (lane l and lane l ^ 32 hold the two
// key halves of one query row): v_permlane32_swap of (x, copy of x) leaves x[l % 32] and x[l % 32 + 32]
// in the two results of every lane. The copy is opaque: given the same value twice, the compiler treats
// the two results as equal and folds max(r0, r1) to r0.
__device__ __forceinline__ int2 both_halves(float x) {
  int y;
  asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(__builtin_bit_cast(int, x)));
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), y, false, false);
  return make_int2(r[0], r[1]);
}
__device__ __forceinline__ float half_max(float x) {
  const int2 r = both_halves(x);
  return fmaxf(__builtin_bit_cast(float, r.x), __builtin_bit_cast(float, r.y));
}
__device__ __forceinline__ float half_sum(float x) {
  const int2 r = both_halves(x);
  return __builtin_bit_cast(float, r.x) + __builtin_bit_cast(float, r.y);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// two floats -> packed fp16 bits (round to nearest even), element 0 in the low half
__device__ __forceinline__ uint32_t f2h2_bits(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0, x1}, f16x2));
}
// two floats -> packed bf16 bits (round to nearest even), element 0 in the low half
__device__ __forceinline__ uint32_t f2bf2_bits(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0, x1}, bf16x2));
}
__device__ __forceinline__ f32x2 h2_to_f2(uint32_t h) {
  return __builtin_convertvector(__builtin_bit_cast(f16x2, h), f32x2);
}
// Two packed bf16 values -> two packed fp16 values (element 0 in the low half). Exact for magnitudes in
// [2^-14, 65504] (a bf16 significand has 8 bits, fp16's has 11); smaller ones round to fp16's subnormals
// (absolute error <= 2^-25), larger ones become +-inf, which then shows in the output.
__device__ __forceinline__ uint32_t bf2_to_h2(uint32_t b) {
  return f2h2_bits(__uint_as_float(b << 16), __uint_as_float(b & 0xffff0000u));
}
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
// v_mfma_f32_32x32x16_f16, the fp16 form of mfma32 (same operand and accumulator layouts)
__device__ __forceinline__ f32x16 mfma32_f16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// How context keys are addressed: flat (slot = position), page table with a power-of-two page size of at
// least 64 (one table read per tile), per-key slot table (page size P: slot = table[t / P] * P + t % P).
enum { CTX_FLAT = 0, CTX_PAGED = 1, CTX_GATHER = 2 };

// Request of scheduling rank rho: requests ordered by context length, longest first (ties by index),
// so that the longest workgroups start first and the short ones fill in behind them.
__device__ __forceinline__ int request_of_rank(const int64_t* ctx_lens, int bs, int rho) {
  const int lane = threadIdx.x & 63;
  for (int base = 0; base < bs; base += 64) {
    const int b = base + lane;
    int rank = -1;
    if (b < bs) {
      const int64_t cb = ctx_lens[b];
      rank = 0;
      for (int j = 0; j < bs; ++j) {
        const int64_t cj = ctx_lens[j];
        rank += (cj > cb || (cj == cb && j < b)) ? 1 : 0;
      }
    }
    const uint64_t hit = __builtin_amdgcn_ballot_w64(rank == rho);
    if (hit) return base + __builtin_ctzll(hit);
  }
  return rho;
}

template <int CTX, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void mode_attn_kernel(AttnArgs a) {
  static_assert(NW == 4 || NW == 8, "workgroups of 4 or 8 waves");
  constexpr int LPW = 16 / NW;  // direct loads per wave and tile (1 KB each)
  constexpr int KPW = 64 / NW;  // keys per wave and tile
  // vector table loads per lane issued after each ring refill (the paged layout reads its table with
  // scalar loads)
  constexpr int NT = CTX == CTX_GATHER ? 2 : 0;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int KL = a.K * a.L;
  // argument fields used inside the lambdas below, as locals (a lambda capturing the argument struct
  // itself would force a private-memory copy of it)
  const int kc_ss = a.kc_ss, vc_ss = a.vc_ss, kn_st = a.kn_st, vn_st = a.vn_st;
  const int page_shift = a.page_shift, page_size = a.page_size;
  const int Lb = a.L;
  const bool causal = a.causal != 0;
  const float scale_log2 = a.scale_log2;

  // ---- workgroup -> (request, KV head, split, unit group). A program p = (rank, KV head, split) runs
  //      on XCD p % 8 (workgroup id modulo 8), and its unit groups are consecutive there, so the groups
  //      that read the same K / V run together and share that XCD's L2.
  const int P = a.bs * a.Hkv * a.S;
  const int NG = a.ngroups;
  const int id = blockIdx.x;
  const int jx = id >> 3;
  const int ug = jx % NG;
  const int pidx = (jx / NG) * 8 + (id & 7);
  if (pidx >= P) return;
  const int s = pidx % a.S;
  const int bk = pidx / a.S;
  const int kvh = bk % a.Hkv;
  const int rho = bk / a.Hkv;
  const int b = __builtin_amdgcn_readfirstlane((a.ctx_lens && a.bs > 1) ? request_of_rank(a.ctx_lens, a.bs, rho) : rho);

  const int upr = (KL + UROWS - 1) / UROWS;  // units per query head (the last one padded when KL % 32 != 0)
  const int U = a.G * upr;
  const int u_raw = ug * NW + w;
  const bool active = u_raw < U;           // an idle wave computes a copy of the last unit and stores nothing
  const int u = active ? u_raw : U - 1;
  const int g = u / upr;
  const int head = kvh * a.G + g;
  const int qi_raw = (u % upr) * UROWS + l32;
  // a padding row of the last unit computes a copy of the head's last query (loads stay inside the request)
  // and stores nothing
  const bool row_ok = active && qi_raw < KL;
  const int qi = qi_raw < KL ? qi_raw : KL - 1;  // this lane's query row
  const int token = b * KL + qi;
  const int mode_lo = (qi / a.L) * a.L;    // first block key of this query's mode
  const int tpos = qi - mode_lo;

  // Q^T fragments: B operand, k = d = 16c + 8 half + e
  bf16x8 qf[D / 16];
  {
    const uint16_t* qp = a.q + (int64_t)token * a.q_st + (int64_t)head * a.q_sh + half * 8;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qf[c] = as_bf16x8(*reinterpret_cast<const u16x8*>(qp + c * 16));
  }

  const int ctx = __builtin_amdgcn_readfirstlane(a.ctx_lens ? (int)a.ctx_lens[b] : a.ctx_const);
  const int64_t trow = a.req_idx ? a.req_idx[b] : b;
  // one pass (S = 1): the whole context, then the block tiles. Split (S = SC + 1 partials): partial s < SC
  // takes a range of whole context tiles, partial SC only the block tiles (so that the block work is not
  // added to the critical path of a context split)
  int lo = 0, hi = ctx;
  int n_blk_tiles = (KL + TK - 1) / TK;
  if (a.S > 1) {
    if (s < a.SC) {
      const int per = (ctx + a.SC - 1) / a.SC;
      const int chunk = max(TK, (per + TK - 1) / TK * TK);
      lo = min(s * chunk, ctx);
      hi = min(lo + chunk, ctx);
      n_blk_tiles = 0;
    } else {
      lo = hi = ctx;
    }
  }
  const int n_ctx_tiles = (hi - lo + TK - 1) / TK;
  const int ntiles = n_ctx_tiles + n_blk_tiles;
  if (ntiles == 0) {  // an empty split (more splits than context tiles): contributes nothing
    if (row_ok && a.S > 1 && half == 0) {
      const int64_t nrows = (int64_t)a.bs * a.H * KL;
      a.ws_lse[(int64_t)s * nrows + ((int64_t)b * a.H + head) * KL + qi] = -INFINITY;
    }
    return;
  }
  const int last = ntiles - 1;

  // ---- direct-to-LDS tile loads. Instruction i (0 .. LPW - 1) of wave w fills the 16-byte chunk positions
  //      (LPW w + i) * 64 + lane of a tile: key r = KPW w + 4 i + lane / 16, chunk position lane % 16.
  //      Keys past the end of a tile's range are clamped to its last valid key (that row is read again
  //      and gets probability 0 in the softmax), so every lane always issues its loads.
  const int pc = lane & 15;
  const int rsub = lane >> 4;
  const int v_col = (pc ^ (rsub << 2)) * 8;
  auto k_col = [&](int r) __attribute__((always_inline)) { return (pc ^ (r & 15)) * 8; };  // key r's chunk
  const int32_t* trow_p = a.table ? a.table + trow * a.table_stride : nullptr;
  const uint16_t* kc_h = a.kc + (int64_t)kvh * a.kc_sh;
  const uint16_t* vc_h = a.vc + (int64_t)kvh * a.vc_sh;
  const uint16_t* kn_h = a.kn + (int64_t)b * KL * a.kn_st + (int64_t)kvh * a.kn_sh;
  const uint16_t* vn_h = a.vn + (int64_t)b * KL * a.vn_st + (int64_t)kvh * a.vn_sh;
  // byte offsets of this lane's LPW rows within a full context tile (uniform-base layouts). Load i reads
  // key r0 + 4 i (r0 = KPW w + lane / 16): the uniform part 4 i * stride goes into the base address, and
  // the K chunk swizzle of key r0 + 4 i is that of r0 with bit 2 of the chunk index flipped by i
  // (r0 % 16 + 4 i < 16, so no carry), which keeps two lane offsets live instead of 2 LPW.
  const int r0k = KPW * w + rsub;
  const uint32_t offk0 = (uint32_t)(r0k * kc_ss + k_col(r0k)) * 2u;
  const uint32_t offv0 = (uint32_t)(r0k * vc_ss + v_col) * 2u;
  const uint32_t lds_b = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)lds_kv;
  auto kslot_byte = [&](int j) __attribute__((always_inline)) { return lds_b + (uint32_t)(j * TILE * 2); };
  auto vslot_byte = [&](int j) __attribute__((always_inline)) { return lds_b + (uint32_t)((KSLOTS + j) * TILE * 2); };

  // table entry a later issue of tile t needs: CTX_PAGED -> the tile's page (uniform; K in lane 0, V in
  // lane 1 of one load), CTX_GATHER -> the slot-table entry of key KPW w + lane % KPW (one load each)
  auto gather_entry = [&](int t) __attribute__((always_inline)) {
    const int kk = max(min(lo + t * TK + KPW * w + (lane & (KPW - 1)), hi - 1), 0);
    return trow_p[page_shift >= 0 ? kk >> page_shift : kk / page_size];
  };
  // page of tile t (uniform): a scalar load (s_load_dword through the constant address space), which is
  // tracked by lgkmcnt and so never waits for the direct-to-LDS loads in flight
  typedef const __attribute__((address_space(4))) int32_t* const_i32p;
  auto page_of_tile = [&](int t) __attribute__((always_inline)) {
    const int idx = __builtin_amdgcn_readfirstlane(max(min(lo + t * TK, hi - 1), 0) >> page_shift);
    return ((const_i32p)trow_p)[idx];
  };
  // issue one tile of K (is_v = false) or V into the LDS slot at lds_byte
  auto issue = [&](bool is_v, int t, uint32_t lds_byte, int32_t entry) __attribute__((always_inline)) {
    const int col_v = v_col;
    if (t < n_ctx_tiles) {
      const int k0 = lo + t * TK;
      const int nv = hi - k0;
      const int ss = is_v ? vc_ss : kc_ss;
      const uint16_t* cache = is_v ? vc_h : kc_h;
      if constexpr (CTX == CTX_GATHER) {
        const int kk = max(min(k0 + KPW * w + (lane & (KPW - 1)), hi - 1), 0);
        const int slot_own = page_shift >= 0 ? (entry << page_shift) + (kk & (page_size - 1))
                                             : entry * page_size + kk % page_size;
        // lane source of load i's slot (key r0 + 4 i) and the key's chunk column: formed here from one
        // value each (kept live across the loop as LPW values apiece, they spill, and every reload drains
        // the direct loads in flight)
        int src = rsub << 2;
        int kcol = k_col(r0k);
        asm volatile("" : "+v"(src), "+v"(kcol));
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
          const int slot = __builtin_amdgcn_ds_bpermute(src + 16 * i, slot_own);
          const uint16_t* gp = cache + (int64_t)slot * ss + (is_v ? col_v : (kcol ^ (32 * i)));
          dma16(gp, lds_byte + (LPW * w + i) * 1024);
        }
      } else {
        int64_t slot0 = k0;
        if constexpr (CTX == CTX_PAGED) slot0 = ((int64_t)entry << page_shift) + (k0 & (page_size - 1));
        const uint16_t* base = cache + slot0 * ss;
        if (nv >= TK) {
#pragma unroll
          for (int i = 0; i < LPW; ++i) {
            const uint32_t offk = offk0 + (uint32_t)(4 * i * kc_ss) * 2u +
                                  (uint32_t)(((k_col(r0k) ^ (32 * i)) - k_col(r0k)) * 2);
            dma16_s(base + 4 * i * (is_v ? vc_ss : 0), is_v ? offv0 : offk, lds_byte + (LPW * w + i) * 1024);
          }
        } else {
#pragma unroll
          for (int i = 0; i < LPW; ++i) {
            const int r0 = KPW * w + 4 * i + rsub;
            const int r = min(r0, nv - 1);
            dma16_s(base, (uint32_t)(r * ss + (is_v ? col_v : k_col(r0))) * 2u, lds_byte + (LPW * w + i) * 1024);
          }
        }
      }
    } else {
      const int b0 = (t - n_ctx_tiles) * TK;
      const int nv = KL - b0;
      const int st = is_v ? vn_st : kn_st;
      const uint16_t* base = (is_v ? vn_h : kn_h) + (int64_t)b0 * st;
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int r0 = KPW * w + 4 * i + rsub;
        const int r = min(r0, nv - 1);
        dma16_s(base, (uint32_t)(r * st + (is_v ? col_v : k_col(r0))) * 2u, lds_byte + (LPW * w + i) * 1024);
      }
    }
  };

  // per-lane LDS offsets (elements) of the MFMA operands. K row ks * 32 + l32, d chunk 2c + half sits at
  // k_base ^ (c << 4) (+ 4096 for ks = 1): the swizzled chunk index is (2c + half) ^ (l32 & 15).
  // V^T fragment (d block db, 16-key chunk c): v_base ^ (db << 5), + 2048 c (+ 1024 for the second
  // 4-key group); the swizzled chunk index is (4 db + 2 (group & 1) + (sl & 3) / 2) ^ (sw << 2).
  // Slot offsets are multiples of TILE, above every bit the XORs touch.
  const int k_base = l32 * 128 + ((((half ^ l32) & 1) | (l32 & 14)) << 3);
  int v_base;
  {
    const int grp = lane >> 4, sl = lane & 15, sw = sl >> 2;
    v_base = (4 * half + sw) * 128 + (sw << 5) + (2 * (grp & 1) + ((sl & 3) >> 1)) * 8 + (sl & 1) * 4;
  }

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 oacc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) oacc[db] = (f32x16){};

  // S^T of one tile (K in slot kslot): keys 32 ks + 8 (r / 4) + 4 half + r % 4, column = this lane's query
  auto scores = [&](int kslot, f32x16 (&sv)[2]) __attribute__((always_inline)) {
    const int kb = k_base + kslot * TILE;
    f32x16 acc0 = {}, acc1 = {};
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const int off = kb ^ (c << 4);
      const u16x8 k0f = *reinterpret_cast<const u16x8*>(lds_kv + off);
      const u16x8 k1f = *reinterpret_cast<const u16x8*>(lds_kv + off + 32 * 128);
      acc0 = mfma32(as_bf16x8(k0f), qf[c], acc0);
      acc1 = mfma32(as_bf16x8(k1f), qf[c], acc1);
    }
    sv[0] = acc0;
    sv[1] = acc1;
  };
  // online softmax of tile t, part 1: masking, row max and the lazy rescale; returns the reference the
  // probabilities are taken against
  auto softmax_max = [&](int t, f32x16 (&sv)[2]) __attribute__((always_inline)) {
    const bool is_ctx = t < n_ctx_tiles;
    // valid keys of this tile: [klo, khi) in tile coordinates; only the last context tile and the
    // block tiles (mode mask) need masking
    int klo = 0, khi = hi - (lo + t * TK);
    if (!is_ctx) {
      const int base = (t - n_ctx_tiles) * TK;
      klo = mode_lo - base;
      khi = mode_lo + (causal ? tpos + 1 : Lb) - base;
    }
    if (!is_ctx || khi < TK) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = ks * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          sv[ks][r] = (key >= klo && key < khi) ? sv[ks][r] : -INFINITY;
        }
    }
    // row max of the raw scores (the scale is positive, so it commutes with max)
    float tmax = -INFINITY;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sv[ks][r]);
    tmax = half_max(tmax);
    const float tm = tmax * scale_log2;
    // lazy rescale: the running reference m_run moves only when a score exceeds it by more than 8
    // (probabilities stay below 2^8, well inside fp16's range); any reference gives the same softmax
    if (__builtin_amdgcn_ballot_w64(tm > m_run + 8.f) != 0) {
      const float m_new = fmaxf(m_run, tm);
      const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) oacc[db] *= alpha;
      m_run = m_new;
    }
    return (m_run == -INFINITY) ? 0.f : m_run;
  };
  // V tile in V slot j: bf16 -> fp16 in place, element-wise (the swizzle does not matter). Each wave widens
  // the 16 / NW KB that its own direct loads filled (slot bytes 1024 LPW w .. + 1024 LPW - 1, 16 bytes per lane per
  // load), so its own vmcnt wait is all it needs before, and the next workgroup barrier publishes the result.
  auto widen_v = [&](int j) __attribute__((always_inline)) {
    u32x4* vs = reinterpret_cast<u32x4*>(lds_kv + (KSLOTS + j) * TILE) + 64 * LPW * w + lane;
    u32x4 x[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) x[i] = vs[64 * i];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      u32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t u = x[i][e];
        y[e] = bf2_to_h2(u);
      }
      vs[64 * i] = y;
    }
  };

  // ---- ring: K of tile t in K slot t % 3, V of tile t in V slot t % 2. Iteration t issues K(t + 3) right
  //      after its first barrier (K slot t % 3 was last read in iteration t - 1; the per-key gather layout
  //      issues it at the end instead) and V(t + 2) after its second barrier, then the gather layout's
  //      table entries for the next refill. The top of iteration t needs K(t + 1) and V(t), issued in
  //      iteration t - 2; at most 8 + NT loads issued after V(t) are then outstanding. Tile indices past
  //      the end are clamped (a harmless reload into a slot nobody reads again).
  int32_t ek = 0, ev = 0;  // CTX_GATHER: slot-table entries for the next refill
  {
    // prologue: K(0); K(1), V(0); K(2), V(1) -- entries read up front
    int32_t e[5] = {0, 0, 0, 0, 0};
    const int tk[5] = {0, min(1, last), min(2, last), 0, min(1, last)};
    if constexpr (CTX == CTX_PAGED) {
#pragma unroll
      for (int x = 0; x < 5; ++x) e[x] = page_of_tile(tk[x]);
    } else if constexpr (CTX == CTX_GATHER) {
#pragma unroll
      for (int x = 0; x < 5; ++x) e[x] = gather_entry(tk[x]);
    }
    // Q's loads (issued above) may still be in flight: every wait below counts from the youngest load, and
    // Q's are older than any direct load, so they are covered by the first one; the paged / gather layouts
    // read their table entries first (a compiler-issued load younger than the direct loads would shift the
    // counts), so for them everything is drained here
    if constexpr (CTX != CTX_FLAT) wait_vmcnt<0>();
    issue(false, 0, kslot_byte(0), e[0]);
    issue(false, tk[1], kslot_byte(1), e[1]);
    issue(true, 0, vslot_byte(0), e[3]);
    issue(false, tk[2], kslot_byte(2), e[2]);
    issue(true, tk[4], vslot_byte(1), e[4]);
    if constexpr (CTX == CTX_GATHER) {
      ek = gather_entry(min(3, last));
      ev = gather_entry(min(2, last));
    }
  }
  f32x16 s_a[2], s_b[2];
  wait_vmcnt<4 * LPW + NT>();  // K(0) has landed
  block_barrier();
  scores(0, s_a);
  wait_vmcnt<2 * LPW + NT>();  // K(1) and V(0) have landed
  widen_v(0);
  wait_lgkmcnt0();
  block_barrier();  // K(1) and the widened V(0) are visible, and every wave is done with K slot 0

  // The 32 MFMAs of an iteration run as a fixed sequence of slots: slot s < 8 is S^T subtile 0 of tile
  // t + 1 (d chunk s), 8..15 P V of key chunks 0 and 1 of tile t (d block s % 4), 16..23 S^T subtile 1,
  // 24..31 P V of key chunks 2 and 3. Each slot's LDS operand is read FD slots ahead (the reads' latency
  // overlaps the MFMAs in between), and the probabilities of tile t are formed one key pair per slot in
  // slots 0..7 (keys 0..31) and 16..23 (keys 32..63), each chunk before its P V slots. A scheduling
  // barrier closes every slot so that the compiler keeps this order (it otherwise hoists all the reads
  // and runs out of registers, or sinks them next to their MFMAs).
  constexpr int FD = 2;
  auto slot_is_qk = [](int sl) __attribute__((always_inline)) { return sl < 8 || (sl >= 16 && sl < 24); };
  auto fetch = [&](int sl, int kb, int vb) __attribute__((always_inline)) {
    u32x4 r;
    if (slot_is_qk(sl)) {
      const int ks = sl >= 16 ? 1 : 0, cc = sl & 7;
      r = *reinterpret_cast<const u32x4*>(lds_kv + ((kb ^ (cc << 4)) + ks * 32 * 128));
    } else {
      const int c = sl < 12 ? 0 : sl < 16 ? 1 : sl < 28 ? 2 : 3, db = sl & 3;
      const int v_off = (vb ^ (db << 5)) + 2048 * c;
      const v4i16 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(lds_kv + v_off));
      const v4i16 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(lds_kv + v_off + 1024));
      const v4i16 va8[2] = {x0, x1};
      r = __builtin_bit_cast(u32x4, va8);
    }
    return r;
  };
  auto iteration = [&](int t, f32x16 (&s_cur)[2], f32x16 (&s_nxt)[2]) __attribute__((always_inline)) {
    const int k1 = (t + 1) % KSLOTS;
    const int v0 = t & 1;
    if constexpr (CTX != CTX_GATHER) {
      // K slot t % 3 held K(t), last read in iteration t - 1: refill it now, overlapping this iteration
      issue(false, min(t + 3, last), kslot_byte(t % KSLOTS), CTX == CTX_PAGED ? page_of_tile(min(t + 3, last)) : 0);
    }
    const float msub = softmax_max(t, s_cur);
    const int kb = k_base + k1 * TILE;
    const int vb = v_base + (KSLOTS + v0) * TILE;
    u32x4 opnd[32];
#pragma unroll
    for (int sl = 0; sl < FD; ++sl) opnd[sl] = fetch(sl, kb, vb);
    u32x4 pv[4];  // P^T B fragments (fp16 pairs) of the four 16-key chunks
    float psum = 0.f;
    f32x16 acc0 = {}, acc1 = {};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int sl = 0; sl < 32; ++sl) {
      if (sl + FD < 32) opnd[sl + FD] = fetch(sl + FD, kb, vb);
      if (slot_is_qk(sl)) {
        if (sl < 8) acc0 = mfma32(__builtin_bit_cast(bf16x8, opnd[sl]), qf[sl & 7], acc0);
        else acc1 = mfma32(__builtin_bit_cast(bf16x8, opnd[sl]), qf[sl & 7], acc1);
      } else {
        const int c = sl < 12 ? 0 : sl < 16 ? 1 : sl < 28 ? 2 : 3, db = sl & 3;
        oacc[db] = mfma32_f16(__builtin_bit_cast(f16x8, opnd[sl]), __builtin_bit_cast(f16x8, pv[c]), oacc[db]);
      }
      if (slot_is_qk(sl)) {
        // key pair q of chunk c: S^T registers r, r + 1 of subtile c / 2
        const int c = (sl < 8 ? 0 : 2) + ((sl & 7) >> 2), q = sl & 3;
        const int r = (c & 1) * 8 + 2 * q;
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[c >> 1][r], scale_log2, -msub));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[c >> 1][r + 1], scale_log2, -msub));
        psum += p0 + p1;
        // keeps the row-sum add in this slot: left free, the compiler sinks all 32 adds to the end of the
        // iteration as one dependent chain and keeps the probabilities live until then (14 more VGPRs)
        asm volatile("" : "+v"(psum));
        pv[c][q] = f2h2_bits(p0, p1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l_run += psum;
    s_nxt[0] = acc0;
    s_nxt[1] = acc1;
    // K(t + 2) and V(t + 1) have landed (only the loads issued since V(t + 1) may be outstanding: K(t + 3),
    // or with the per-key table the NT entry loads); this wave widens its part of V(t + 1), which nobody
    // reads during this iteration
    wait_vmcnt<CTX == CTX_GATHER ? NT : LPW>();
    if (t + 1 < ntiles) widen_v(v0 ^ 1);
    wait_lgkmcnt0();               // this wave's reads of K slot (t + 1) % 3 and V slot t % 2 have returned
    // every wave is done with V slot t % 2 (and with K slot t % 3 since t - 1); K(t + 2) and the widened
    // V(t + 1) are visible for iteration t + 1
    block_barrier();
    if constexpr (CTX == CTX_GATHER) issue(false, min(t + 3, last), kslot_byte(t % KSLOTS), ek);
    issue(true, min(t + 2, last), vslot_byte(v0), CTX == CTX_PAGED ? page_of_tile(min(t + 2, last)) : ev);
    if constexpr (CTX == CTX_GATHER) {
      ek = gather_entry(min(t + 4, last));
      ev = gather_entry(min(t + 3, last));
    }
  };
  for (int t = 0;;) {
    iteration(t, s_a, s_b);
    if (++t >= ntiles) break;
    iteration(t, s_b, s_a);
    if (++t >= ntiles) break;
  }
  wait_vmcnt<0>();  // no direct-to-LDS load may outlive the workgroup

  // A V value beyond fp16's range became an infinity in a widened tile: every accumulator column it touched is
  // non-finite (inf P, or 0 inf = NaN for a masked key), in every wave. The workgroup then computes its tiles
  // again, one at a time through K slot 0 and V slot 0, with V left in bf16 and the P V product in bf16. The
  // waves' verdicts meet in K slot 2 (no further shared memory: one more word would keep a second workgroup of
  // four waves off the CU), once every wave's ring reads and direct loads are done; that slot is not refilled.
  // (x 0 is 0 for a finite x and NaN otherwise: one FMA per accumulator, four chains)
  float zz[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) zz[r & 3] = __builtin_fmaf(oacc[db][r], 0.f, zz[r & 3]);
  const bool nonfinite = !__builtin_isfinite((zz[0] + zz[1]) + (zz[2] + zz[3]));
  volatile uint32_t* const verdict = reinterpret_cast<volatile uint32_t*>(lds_kv + 2 * TILE);
  block_barrier();
  if (lane == 0) verdict[w] = __builtin_amdgcn_ballot_w64(nonfinite) != 0 ? 1u : 0u;
  wait_lgkmcnt0();
  block_barrier();
  uint32_t any_nonfinite = 0;
#pragma unroll
  for (int x = 0; x < NW; ++x) any_nonfinite |= verdict[x];
  if (any_nonfinite) {
    m_run = -INFINITY;
    l_run = 0.f;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) oacc[db] = (f32x16){};
    for (int t = 0; t < ntiles; ++t) {
      int32_t e = 0;
      if constexpr (CTX == CTX_PAGED) e = page_of_tile(t);
      else if constexpr (CTX == CTX_GATHER) e = gather_entry(t);
      if (t > 0) block_barrier();  // every wave is done with the slots' previous tile
      issue(false, t, kslot_byte(0), e);
      issue(true, t, vslot_byte(0), e);
      wait_vmcnt<0>();
      block_barrier();
      // scores as in the ring loop, one d chunk at a time (this path is rare: registers, not latency, matter)
      f32x16 sv[2] = {{}, {}};
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        const int off = k_base ^ (c << 4);
        const u16x8 k0f = *reinterpret_cast<const u16x8*>(lds_kv + off);
        const u16x8 k1f = *reinterpret_cast<const u16x8*>(lds_kv + off + 32 * 128);
        sv[0] = mfma32(as_bf16x8(k0f), qf[c], sv[0]);
        sv[1] = mfma32(as_bf16x8(k1f), qf[c], sv[1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      const float msub = softmax_max(t, sv);
      // per 16-key chunk c: the probabilities of its key pairs q (S^T registers r, r + 1 of subtile c / 2) split
      // into bf16 hi + lo pairs (P to about 2^-17; V is exact in bf16), then its P V products
      const int vb = v_base + KSLOTS * TILE;
      float psum = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        u32x4 ph, pl;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = (c & 1) * 8 + 2 * q;
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[c >> 1][r], scale_log2, -msub));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[c >> 1][r + 1], scale_log2, -msub));
          psum += p0 + p1;
          ph[q] = f2bf2_bits(p0, p1);
          const f32x2 hf = {__uint_as_float(ph[q] << 16), __uint_as_float(ph[q] & 0xffff0000u)};
          pl[q] = f2bf2_bits(p0 - hf[0], p1 - hf[1]);
        }
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          const bf16x8 vf = __builtin_bit_cast(bf16x8, fetch((c < 2 ? 8 + 4 * c : 16 + 4 * c) + db, 0, vb));
          oacc[db] = mfma32(vf, __builtin_bit_cast(bf16x8, ph), oacc[db]);
          oacc[db] = mfma32(vf, __builtin_bit_cast(bf16x8, pl), oacc[db]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      l_run += psum;
    }
    wait_lgkmcnt0();
  }
  if (!active) return;

  const float l_tot = half_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  // the row indices again, opaque to the compiler: it would otherwise keep their 64-bit forms from the Q
  // loads live across the tile loops
  int token_e = token, qi_e = qi;
  asm volatile("" : "+v"(token_e), "+v"(qi_e));
  if (a.S == 1) {
    if (!row_ok) return;
    uint16_t* op = a.out + (int64_t)token_e * a.o_st + (int64_t)head * a.o_sh;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = db * 32 + gq * 8 + half * 4;
        const u16x4 vals = {f2bf_bits(oacc[db][gq * 4 + 0] * inv), f2bf_bits(oacc[db][gq * 4 + 1] * inv),
                            f2bf_bits(oacc[db][gq * 4 + 2] * inv), f2bf_bits(oacc[db][gq * 4 + 3] * inv)};
        *reinterpret_cast<u16x4*>(op + d0) = vals;
      }
  } else {
    // partial output row in fp16, scaled by a power of two into (-1, 1): half the bytes of fp32 for the
    // merge to read back, at 2^-12 of the row's largest value (the bf16 output's own rounding is 2^-9)
    const int64_t prow = ((int64_t)b * a.H + head) * KL + qi_e;
    const int64_t nrows = (int64_t)a.bs * a.H * KL;
    float mx = 0.f;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fabsf(oacc[db][r] * inv));
    mx = half_max(mx);
    const int ex = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) : 0;  // mx = f 2^ex, f in [0.5, 1)
    const float down = __builtin_ldexpf(inv, -ex);
    if (!row_ok) return;
    uint16_t* op = a.ws_o + ((int64_t)s * nrows + prow) * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = db * 32 + gq * 8 + half * 4;
        u32x2 hv;
        hv[0] = f2h2_bits(oacc[db][gq * 4 + 0] * down, oacc[db][gq * 4 + 1] * down);
        hv[1] = f2h2_bits(oacc[db][gq * 4 + 2] * down, oacc[db][gq * 4 + 3] * down);
        *reinterpret_cast<u32x2*>(op + d0) = hv;
      }
    if (half == 0) {
      a.ws_lse[(int64_t)s * nrows + prow] = l_tot > 0.f ? m_run + __log2f(l_tot) : -INFINITY;
      a.ws_exp[(int64_t)s * nrows + prow] = (float)ex;
    }
  }
}

// one thread per 8 d of one row (16-byte partial loads); 16 threads per row, 16 rows per workgroup. The
// partials of a row are read in batches of 16 splits (all loads of a batch issued before any is used) and
// combined with a running log-sum-exp.
__global__ __launch_bounds__(256) void mode_attn_merge_kernel(AttnArgs a) {
  constexpr int SB = 16;  // partials per batch: all of a batch's loads are in flight together
  const int KL = a.K * a.L;
  const int64_t nrows = (int64_t)a.bs * a.H * KL;
  const int64_t prow = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (prow >= nrows) return;
  const int d0 = (threadIdx.x & 15) * 8;
  float m = -INFINITY, tot = 0.f;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  for (int s0 = 0; s0 < a.S; s0 += SB) {
    float l[SB], ex[SB];
    u32x4 oh[SB];
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int s = s0 + j;
      l[j] = -INFINITY;
      ex[j] = 0.f;
      oh[j] = (u32x4){0u, 0u, 0u, 0u};
      if (s < a.S) {  // uniform
        l[j] = a.ws_lse[s * nrows + prow];
        ex[j] = a.ws_exp[s * nrows + prow];
        oh[j] = *reinterpret_cast<const u32x4*>(a.ws_o + (s * nrows + prow) * D + d0);
      }
    }
    float mb = l[0];
#pragma unroll
    for (int j = 1; j < SB; ++j) mb = fmaxf(mb, l[j]);
    if (mb == -INFINITY) continue;
    const float mn = fmaxf(m, mb);
    const float sc = exp2f(m - mn);  // 0 while m is -inf
    acc0 *= sc;
    acc1 *= sc;
    tot *= sc;
    m = mn;
#pragma unroll
    for (int j = 0; j < SB; ++j)
      if (l[j] != -INFINITY) {  // an empty split wrote no partial output
        const float wgt = exp2f(l[j] - m);
        const float wo = __builtin_ldexpf(wgt, (int)ex[j]);
        const f32x2 o01 = h2_to_f2(oh[j][0]), o23 = h2_to_f2(oh[j][1]);
        const f32x2 o45 = h2_to_f2(oh[j][2]), o67 = h2_to_f2(oh[j][3]);
        acc0 += (f32x4){o01[0], o01[1], o23[0], o23[1]} * wo;
        acc1 += (f32x4){o45[0], o45[1], o67[0], o67[1]} * wo;
        tot += wgt;
      }
  }
  const float inv = tot > 0.f ? 1.f / tot : 0.f;
  const int qi = (int)(prow % KL);
  const int64_t bh = prow / KL;
  const int head = (int)(bh % a.H);
  const int b = (int)(bh / a.H);
  uint16_t* op = a.out + ((int64_t)b * KL + qi) * a.o_st + (int64_t)head * a.o_sh + d0;
  const u16x8 vals = {f2bf_bits(acc0[0] * inv), f2bf_bits(acc0[1] * inv), f2bf_bits(acc0[2] * inv),
                      f2bf_bits(acc0[3] * inv), f2bf_bits(acc1[0] * inv), f2bf_bits(acc1[1] * inv),
                      f2bf_bits(acc1[2] * inv), f2bf_bits(acc1[3] * inv)};
  *reinterpret_cast<u16x8*>(op) = vals;
}

}  // namespace

extern "C" int64_t mfd_mode_attn_workspace_bytes(int bs, int num_modes, int block_size, int H, int num_ctx_splits) {
  if (num_ctx_splits <= 1) return 0;
  // num_ctx_splits context partials plus the block-key partial: fp16 rows, lse and scale exponent
  const int64_t rows = (int64_t)bs * H * num_modes * block_size;
  return (int64_t)(num_ctx_splits + 1) * rows * (D * 2 + 4 + 4);
}

extern "C" int mfd_mode_attn(const uint16_t* q, int64_t q_st, int64_t q_sh, const uint16_t* k_new,
                             const uint16_t* v_new, int64_t kn_st, int64_t kn_sh, int64_t vn_st, int64_t vn_sh,
                             const uint16_t* k_cache, const uint16_t* v_cache, int64_t kc_ss, int64_t kc_sh,
                             int64_t vc_ss, int64_t vc_sh, const int32_t* slot_table, int64_t table_stride,
                             int page_size, const int64_t* req_idx, const int64_t* ctx_lens, int ctx_len_const, int bs,
                             int num_modes, int block_size, int H, int Hkv, int D_, float scale, int causal_in_block,
                             int num_ctx_splits, uint16_t* out, int64_t o_st, int64_t o_sh, float* workspace,
                             int64_t workspace_bytes, void* stream) {
  if (D_ != D) return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_mode_attn: head dim %d (only %d)", D_, D);
  if (bs < 0 || num_modes < 1 || block_size < 1 || H < 1 || Hkv < 1 || H % Hkv != 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: bad sizes bs=%d K=%d L=%d H=%d Hkv=%d", bs, num_modes,
                         block_size, H, Hkv);
  const int KL = num_modes * block_size;
  if (KL > (1 << 16))
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_mode_attn: num_modes * block_size = %d above 65536", KL);
  if (num_ctx_splits < 1 || num_ctx_splits > 1024)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: num_ctx_splits %d (1..1024)", num_ctx_splits);
  if (page_size < 1) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: page_size %d", page_size);
  if (!(scale > 0.f)) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: scale must be positive");
  // per-lane byte offsets inside a 64-key tile are 32-bit: (63 * stride + 127) * 2 < 2^31
  if (kc_ss < 0 || vc_ss < 0 || kn_st < 0 || vn_st < 0 || kc_ss > (1 << 24) || vc_ss > (1 << 24) ||
      kn_st > (1 << 24) || vn_st > (1 << 24))
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "mfd_mode_attn: row / slot strides must be in [0, 2^24] elements");
  if (!ctx_lens && ctx_len_const < 0) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: negative context length");
  if (bs == 0) return MFD_OK;
  if (!q || !k_new || !v_new || !out || ((!k_cache || !v_cache) && (ctx_lens || ctx_len_const > 0)))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: null tensor pointer");
  // every row is moved in 16-byte pieces: 16-byte aligned bases, strides in multiples of 8 elements
  auto mis16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; };
  if (mis16(q) || mis16(k_new) || mis16(v_new) || mis16(out) || mis16(k_cache) || mis16(v_cache) ||
      ((q_st | q_sh | kn_st | kn_sh | vn_st | vn_sh | kc_ss | kc_sh | vc_ss | vc_sh | o_st | o_sh) & 7) != 0)
    return mfd_set_error(MFD_ERR_UNSUPPORTED,
                         "mfd_mode_attn: tensors need 16-byte aligned rows (bases and strides in multiples of 8)");
  const int64_t need = mfd_mode_attn_workspace_bytes(bs, num_modes, block_size, H, num_ctx_splits);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_mode_attn: workspace of %lld bytes needed", (long long)need);
  AttnArgs a{};
  a.q = q; a.q_st = q_st; a.q_sh = q_sh;
  a.kn = k_new; a.vn = v_new; a.kn_st = (int)kn_st; a.kn_sh = kn_sh; a.vn_st = (int)vn_st; a.vn_sh = vn_sh;
  a.kc = k_cache; a.vc = v_cache; a.kc_ss = (int)kc_ss; a.kc_sh = kc_sh; a.vc_ss = (int)vc_ss; a.vc_sh = vc_sh;
  a.table = slot_table; a.table_stride = table_stride; a.page_size = page_size;
  a.req_idx = req_idx; a.ctx_lens = ctx_lens; a.ctx_const = ctx_len_const;
  a.out = out; a.o_st = o_st; a.o_sh = o_sh;
  const int64_t rows = (int64_t)bs * H * KL;
  const int SP = num_ctx_splits > 1 ? num_ctx_splits + 1 : 1;
  a.ws_o = reinterpret_cast<uint16_t*>(workspace);
  a.ws_lse = workspace ? reinterpret_cast<float*>(a.ws_o + (int64_t)SP * rows * D) : nullptr;
  a.ws_exp = workspace ? a.ws_lse + (int64_t)SP * rows : nullptr;
  a.bs = bs; a.K = num_modes; a.L = block_size; a.H = H; a.Hkv = Hkv; a.G = H / Hkv; a.S = SP;
  a.SC = num_ctx_splits;
  a.causal = causal_in_block ? 1 : 0;
  a.scale_log2 = scale * 1.4426950408889634f;
  const int units = a.G * ((KL + UROWS - 1) / UROWS);
  // eight-wave workgroups (one per CU, each K / V tile loaded once per CU for twice the queries) when the
  // units of a KV head come in eights; four-wave ones (two per CU) otherwise
  const int NW = (units % 8 == 0) ? 8 : NWAVES;
  a.ngroups = (units + NW - 1) / NW;
  const int P = bs * Hkv * SP;
  const int P8 = (P + 7) / 8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int mode = CTX_FLAT;
  if (slot_table) {
    // a power-of-two page size turns the per-key page and offset into a shift and a mask
    a.page_shift = (page_size & (page_size - 1)) == 0 ? __builtin_ctz((unsigned)page_size) : -1;
    mode = (page_size >= TK && a.page_shift >= 0) ? CTX_PAGED : CTX_GATHER;
  }
  const dim3 grid(8 * P8 * a.ngroups);
  switch (mode) {
    case CTX_FLAT:
      if (NW == 8) hipLaunchKernelGGL((mode_attn_kernel<CTX_FLAT, 8>), grid, dim3(512), 0, st, a);
      else hipLaunchKernelGGL((mode_attn_kernel<CTX_FLAT, 4>), grid, dim3(256), 0, st, a);
      break;
    case CTX_PAGED:
      if (NW == 8) hipLaunchKernelGGL((mode_attn_kernel<CTX_PAGED, 8>), grid, dim3(512), 0, st, a);
      else hipLaunchKernelGGL((mode_attn_kernel<CTX_PAGED, 4>), grid, dim3(256), 0, st, a);
      break;
    default:
      if (NW == 8) hipLaunchKernelGGL((mode_attn_kernel<CTX_GATHER, 8>), grid, dim3(512), 0, st, a);
      else hipLaunchKernelGGL((mode_attn_kernel<CTX_GATHER, 4>), grid, dim3(256), 0, st, a);
      break;
  }
  MFD_CHECK_LAUNCH();
  if (num_ctx_splits > 1) {
    hipLaunchKernelGGL(mode_attn_merge_kernel, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, st, a);
    MFD_CHECK_LAUNCH();
  }
  return MFD_OK;
}
