// Draft LM-head product of the draft top-k head (DDTreeDraftTopK: logits = hidden @ weight^T over the
// drafted rows, inference/sglang/patches/sglang-v0.5.22-mfd.patch:1523-1532) for gfx950, and the head's
// single entry point (the product, then the logits step of logits_topk.hip on its output).
//
// The product streams the weight (vocabulary x hidden, bf16, read once per 128 drafted rows: 778 MB at a
// 151936-token vocabulary and hidden 2560) against the drafted rows, which every workgroup shares.
//  * The vocabulary is split evenly over the grid's workgroups (one per CU; ranges of a multiple of 8 rows),
//    each taking its range in passes of 128 weight rows against all (up to 128) drafted rows.
//  * Both operands stream through LDS in 64-k stages (128 weight rows and 128 drafted rows, 128 bytes each,
//    32 KB per stage) in a ring of four stages. Two producer waves issue the direct-to-LDS loads (every load
//    instruction moves 8 whole rows x 128 contiguous bytes), up to three stages ahead; four consumer waves
//    split each pass's 128 x 128 outputs 2 x 2, a consumer computing 64 weight rows x 64 drafted rows as
//    4 x 4 v_mfma_f32_16x16x32_bf16 tiles (fp32 accumulators, 64 registers). The waves hand stages over
//    through LDS counters with bounded polling, so the consumers never stall on load issue and the producers
//    never wait for products: each producer counts the stages whose loads it has seen land, each consumer
//    the stages it has released, and a wave waits until every counter of the other side reaches the stage
//    (one shared count could be reached by a wave running two stages ahead while another lags). A wait that
//    runs out (it never should) turns the workgroup's remaining outputs into NaN instead of hanging.
//  * 16-byte chunk c of staged row r sits at slot c ^ ((r >> 1) & 7) of the row, so the 16 lanes of each
//    quarter of an operand read hit distinct banks.
//  * The drafted-row stream restarts at k = 0 for every pass: stage v of a workgroup is pass v / (K / 64),
//    k-chunk v % (K / 64). Rows past the end of a pass (the last one) read the pass's last row; rows past M
//    read row M - 1; neither is stored. A pass's outputs are rounded to bf16 (round to nearest even, as the
//    library GEMM of the reference) and stored when its last stage is done.

#include "mfd_common.h"

namespace {

constexpr int NC = 4;                 // consumer waves (2 x 2 over a pass's outputs)
constexpr int NP = 2;                 // producer waves
constexpr int NT = (NC + NP) * 64;
constexpr int MT = 128;               // drafted rows of one launch
constexpr int PT = 128;               // weight rows per pass
constexpr int KS = 64;                // k per stage
constexpr int SROW = KS * 2;          // bytes of a staged row
constexpr int WBLK = PT * SROW;       // weight block of a stage (16 KB)
constexpr int HBLK = MT * SROW;       // drafted-row block of a stage (16 KB)
constexpr int SBUF = WBLK + HBLK;     // a stage: weight block, then drafted-row block
constexpr int NBUF = 4;               // stages in the ring (128 KB)
constexpr int DPW = WBLK / 1024 / NP; // 1-KB weight loads per producer per stage (8)
constexpr int DPH = HBLK / 1024 / NP; // 1-KB drafted-row loads per producer per stage (8)
constexpr int SMEM = NBUF * SBUF + 48;  // + the hand-over counters (16-byte aligned groups) and the failure flag
constexpr int SPIN = 1 << 22;         // polls before a hand-over wait gives up (about 0.3 s: far beyond any real wait)

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct HeadArgs {
  const uint16_t* hidden;  // drafted row m at hidden + (m / rpg) * group_stride + (m % rpg) * row_stride
  int64_t row_stride, group_stride;
  int rpg;
  int row0;                // the launch's drafted rows are row0 .. row0 + M - 1
  const uint16_t* w;       // [N][K] row-major
  uint16_t* out;           // [M][out_stride], row 0 = drafted row row0
  int64_t out_stride;
  int M, N, K;
  int nwg;                 // workgroups of the grid
};

// First vocabulary row of workgroup g: an even split of N rows over nwg workgroups, rounded down to a multiple
// of 8 (non-decreasing in g; workgroup nwg starts at N).
__host__ __device__ __forceinline__ int wg_row0(int g, int N, int nwg) {
  return g >= nwg ? N : (int)(((int64_t)g * N / nwg) & ~(int64_t)7);
}

// One direct-to-LDS load (global_load_lds_dwordx4): lane l's 16 bytes at base + off land at LDS byte address
// lds_byte + 16 l (base and lds_byte wave-uniform). Inline asm: the compiler does not count it among its own
// loads; the producer waits for it explicitly.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds_byte) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds_byte);
  const uint64_t bb = (uint64_t)(uintptr_t)base;
  const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(bb >> 32)) << 32) |
                      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)bb);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(off), "s"(bs) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until each of the NCNT (2 or 4) LDS counters at c (16-byte aligned, read together) reaches target.
// Bounded: a wait that runs out (it never should) sets the workgroup's failure flag and returns, so the kernel
// always completes and the workgroup's remaining outputs are written as NaN instead of values computed from
// stale operands.
template <int NCNT>
__device__ __forceinline__ void wait_all(const int* c, int target, int* fail) {
  static_assert(NCNT == 2 || NCNT == 4, "counter groups of 2 or 4");
  for (int it = 0; it < SPIN; ++it) {
    int lo;
    // through an LDS pointer: a generic (flat) load would also wait for the wave's global loads in flight
    if constexpr (NCNT == 2) {
      const u32x2 x = *(const __attribute__((address_space(3))) volatile u32x2*)c;
      lo = min((int)x[0], (int)x[1]);
    } else {
      const u32x4 x = *(const __attribute__((address_space(3))) volatile u32x4*)c;
      lo = min(min((int)x[0], (int)x[1]), min((int)x[2], (int)x[3]));
    }
    if (__builtin_amdgcn_readfirstlane(lo) >= target) {
      // LDS performs a wave's operations in issue order, so the stage reads (or direct-to-LDS loads) issued
      // after this poll follow it; only the compiler must not move them above it (a workgroup-scope acquire
      // fence would also wait for the producer's loads in flight)
      asm volatile("" ::: "memory");
      return;
    }
    // no sleep between polls: a hand-over is due within a few hundred cycles, and sleeping measured slower
  }
  if ((threadIdx.x & 63) == 0) __atomic_store_n(fail, 1, __ATOMIC_RELAXED);
}
__device__ __forceinline__ void signal_count(int* c) {
  if ((threadIdx.x & 63) == 0) __atomic_fetch_add(c, 1, __ATOMIC_RELEASE);
}
// A consumer's release of a stage: LDS performs a wave's operations in issue order, so a counter update issued
// after the stage's reads lands after them; no wait for the reads' data is needed.
__device__ __forceinline__ void signal_after_reads(int* c) {
  asm volatile("" ::: "memory");
  if ((threadIdx.x & 63) == 0) __atomic_fetch_add(c, 1, __ATOMIC_RELAXED);
}

__global__ __launch_bounds__(NT) void draft_head_kernel(HeadArgs a) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  int* ready = reinterpret_cast<int*>(smem + NBUF * SBUF);  // [NP]: stages producer p has seen land
  int* done = ready + 4;                                     // [NC]: stages consumer c has released
  int* fail = ready + 8;                                     // set by a hand-over wait that ran out
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int R0 = wg_row0(blockIdx.x, a.N, a.nwg);
  const int rows = wg_row0(blockIdx.x + 1, a.N, a.nwg) - R0;
  if (rows <= 0) return;
  const int K = a.K;
  const int SK = K / KS;                   // stages per pass
  const int npass = (rows + PT - 1) / PT;
  const int S = npass * SK;
  if (tid < 9) ready[tid] = 0;
  __syncthreads();

  if (w >= NC) {
    // ---------------------------------------------------------- producer p: half of each block's rows
    const int p = w - NC;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
    // load i fills block rows 64 p + 8 i + lane / 8 (weight and drafted-row blocks alike), at slot lane % 8
    // (chunk (lane % 8) ^ ((row >> 1) & 7))
    uint32_t hoff[DPH], wrow[DPW], wchunk[DPW], woff[DPW];
#pragma unroll
    for (int i = 0; i < DPH; ++i) {
      const int row = 64 * p + 8 * i + (lane >> 3);
      const int c = (lane & 7) ^ ((row >> 1) & 7);
      const int m = a.row0 + min(row, a.M - 1);
      hoff[i] = (uint32_t)(((int64_t)(m / a.rpg) * a.group_stride + (int64_t)(m % a.rpg) * a.row_stride + 8 * c) * 2);
    }
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
      const int row = 64 * p + 8 * i + (lane >> 3);
      wrow[i] = (uint32_t)row;
      wchunk[i] = (uint32_t)(16 * ((lane & 7) ^ ((row >> 1) & 7)));
    }
    int lp = -1, lkc = SK - 1;
    const uint16_t* wp = a.w;
    for (int v = 0; v < S; ++v) {
      if (++lkc == SK) {  // next pass: its weight rows, the last one repeated past the range
        lkc = 0;
        ++lp;
        wp = a.w + ((int64_t)R0 + (int64_t)PT * lp) * K;
        const int last = min(PT, rows - PT * lp) - 1;
#pragma unroll
        for (int i = 0; i < DPW; ++i) woff[i] = (uint32_t)min((int)wrow[i], last) * (uint32_t)(2 * K) + wchunk[i];
      }
      // publish stage v - (NBUF - 1) as soon as it has landed (at most NBUF - 2 later stages in flight),
      // before waiting for the slot of stage v, so a slow slot never delays a ready stage
      if (v >= NBUF - 1) {
        wait_vmcnt<(DPW + DPH) * (NBUF - 2)>();
        signal_count(ready + p);
      }
      if (v >= NBUF) wait_all<NC>(done, v - NBUF + 1, fail);  // every consumer has released the slot's last stage
      const uint32_t dst = lds0 + (uint32_t)(v % NBUF) * SBUF;
      const uint32_t kb = (uint32_t)lkc * SROW;
#pragma unroll
      for (int i = 0; i < DPW; ++i) dma16(wp, woff[i] + kb, dst + (uint32_t)(64 * p) * SROW + 1024u * i);
#pragma unroll
      for (int i = 0; i < DPH; ++i) dma16(a.hidden, hoff[i] + kb, dst + WBLK + (uint32_t)(64 * p) * SROW + 1024u * i);
    }
    wait_vmcnt<0>();
    for (int v = max(S - (NBUF - 1), 0); v < S; ++v) signal_count(ready + p);
    return;
  }

  // -------------------------------------------------------------------- consumer: outputs 64 wa .., 64 wb ..
  const int wa = w & 1, wb = w >> 1;
  const int l16 = lane & 15, g4 = lane >> 4;
  // operand fragments of step st: row (block row base) + l16, chunk 4 st + g4
  uint32_t boff[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) boff[st] = (uint32_t)(l16 * SROW + (((4 * st + g4) ^ ((l16 >> 1) & 7)) << 4));

  f32x4 acc[4][4];
#pragma unroll
  for (int o = 0; o < 4; ++o)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[o][j] = (f32x4){};
  auto read_ops = [&](int v, int st, bf16x8 (&fa)[4], bf16x8 (&fb)[4]) __attribute__((always_inline)) {
    const uint8_t* base = smem + (v % NBUF) * SBUF;
#pragma unroll
    for (int o = 0; o < 4; ++o)
      fa[o] = *reinterpret_cast<const bf16x8*>(base + (64 * wa + 16 * o) * SROW + boff[st]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      fb[j] = *reinterpret_cast<const bf16x8*>(base + WBLK + (64 * wb + 16 * j) * SROW + boff[st]);
  };
  auto mfma16x16 = [&](const bf16x8 (&fa)[4], const bf16x8 (&fb)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[o][j] = mfma16(fa[o], fb[j], acc[o][j]);
  };
  // C register r of accumulator (o, j): weight row 64 wa + 16 o + 4 g4 + r of the pass, drafted row
  // 64 wb + 16 j + l16
  auto epilogue = [&](int pass) __attribute__((always_inline)) {
    const int nloc = PT * pass + 64 * wa + 4 * g4;  // the lane's first row within the workgroup's range
    const bool failed = __builtin_amdgcn_readfirstlane(__atomic_load_n(fail, __ATOMIC_RELAXED)) != 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = 64 * wb + 16 * j + l16;
      if (m < a.M) {
        uint16_t* orow = a.out + (int64_t)m * a.out_stride + R0;
#pragma unroll
        for (int o = 0; o < 4; ++o) {
          const int n = nloc + 16 * o;
          const f32x4 c = acc[o][j];
          u32x2 pk = {__builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){c[0], c[1]}, bf16x2)),
                      __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){c[2], c[3]}, bf16x2))};
          if (failed) pk = (u32x2){0x7FC07FC0u, 0x7FC07FC0u};  // bf16 quiet NaNs
          if (n + 4 <= rows) {
            *reinterpret_cast<u32x2*>(orow + n) = pk;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < rows) orow[n + e] = (uint16_t)(pk[e >> 1] >> (16 * (e & 1)));
          }
        }
      }
    }
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[o][j] = (f32x4){};
  };

  // Stage v: step 1's operands are read while step 0's products run; then, once stage v + 1 has landed, its
  // step-0 operands are read while step 1's products run (the last stage reads an unused slot instead, never
  // used); stage v is released once all of its reads are issued. Two register sets alternate for the step-0
  // operands (unrolled by two).
  bf16x8 fa0[2][4], fb0[2][4], fa1[4], fb1[4];
  wait_all<NP>(ready, 1, fail);
  read_ops(0, 0, fa0[0], fb0[0]);
  int ckc = 0, cp = 0;  // pass and k-chunk of the stage computed
  auto stage = [&](int v, int par) __attribute__((always_inline)) {
    read_ops(v, 1, fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    mfma16x16(fa0[par], fb0[par]);
    __builtin_amdgcn_sched_barrier(0);
    wait_all<NP>(ready, min(v + 2, S), fail);
    read_ops(v + 1, 0, fa0[par ^ 1], fb0[par ^ 1]);
    __builtin_amdgcn_sched_barrier(0);
    mfma16x16(fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    signal_after_reads(done + w);
    if (++ckc == SK) {
      epilogue(cp);
      ckc = 0;
      ++cp;
    }
  };
  int v = 0;
  for (; v + 1 < S; v += 2) {
    stage(v, 0);
    stage(v + 1, 1);
  }
  if (v < S) stage(v, 0);
}


// ---- Wide form, for workgroup ranges of more than one 128-row pass (the full vocabulary). The pass form reads
//      all drafted rows again for every pass, so at 600 weight rows per workgroup the per-CU load path carries
//      the drafted rows 4.7 times next to the weight; here every workgroup holds accumulators for its whole
//      range (up to WRMAX rows) and streams k once, so the drafted rows pass through it once.
//  * Eight waves (two per SIMD); wave w owns weight rows 80 w .. 80 w + 79 of the range (5 tiles of 16) against
//    all 128 drafted rows (8 tiles): 40 v_mfma_f32_16x16x32_bf16 accumulators (160 registers).
//  * Stages of 32 k (one MFMA depth): the range's weight rows and the drafted rows, 64 bytes each (48 KB), in a
//    ring of three; every wave issues its own direct-to-LDS loads (its 80 weight rows and 16 drafted rows: six
//    1-KB loads per stage), stage v + 2 going out once the barrier of stage v has freed its slot.
//  * 16-byte chunk c of staged row r sits at position c ^ ((r >> 2) & 3), so the 16 rows of a fragment read hit
//    distinct banks; a load's lane l fills row l / 4 of its 16 rows at position l % 4.
namespace wide {
constexpr int NW = 8;
constexpr int NTH = NW * 64;
constexpr int VTW = 5;                   // 16-row weight tiles per wave
constexpr int WRMAX = NW * VTW * 16;     // weight rows per workgroup (640)
constexpr int MTL = MT / 16;             // drafted-row tiles (8)
constexpr int KSW = 32;                  // k per stage
constexpr int RB = KSW * 2;              // bytes of a staged row (64)
constexpr int WBW = WRMAX * RB;          // weight block (40 KB)
constexpr int SBW = WBW + MT * RB;       // a stage (48 KB)
constexpr int NBW = 3;                   // ring depth (144 KB)
constexpr int SMEMW = NBW * SBW;
constexpr int LPW = VTW + 1;             // 1-KB loads per wave and stage: VTW weight, 1 drafted
}  // namespace wide

__global__ __launch_bounds__(wide::NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void draft_head_wide_kernel(HeadArgs a) {
  using namespace wide;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int R0 = wg_row0(blockIdx.x, a.N, a.nwg);
  const int rows = wg_row0(blockIdx.x + 1, a.N, a.nwg) - R0;
  if (rows <= 0) return;
  const int K = a.K;
  const int S = K / KSW;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  // load side: lane l fills row (16-row group base) + l / 4 at position l % 4, so it reads chunk
  // (l % 4) ^ ((l / 16) % 4) of that row (the group base is a multiple of 16)
  const int lrow = lane >> 2;
  const int lchunk = (lane & 3) ^ ((lane >> 4) & 3);
  const uint16_t* wbase = a.w + (int64_t)R0 * K;
  uint32_t hoff;
  {
    const int m = a.row0 + min(16 * w + lrow, a.M - 1);
    hoff = (uint32_t)(((int64_t)(m / a.rpg) * a.group_stride + (int64_t)(m % a.rpg) * a.row_stride + 8 * lchunk) * 2);
  }
  // weight tiles of this wave that hold rows of the range (tiles wholly past it are neither loaded nor computed)
  const int vtv = __builtin_amdgcn_readfirstlane(max(0, min(VTW, (rows - VTW * 16 * w + 15) / 16)));
  auto issue = [&](int v) __attribute__((always_inline)) {
    const uint32_t slot = lds0 + (uint32_t)(v % NBW) * SBW;
    const uint32_t kb = (uint32_t)v * RB;
#pragma unroll
    for (int i = 0; i < VTW; ++i) {
      if (i >= vtv) break;
      // tile i of the wave: rows 80 w + 16 i .. ; rows past the range repeat the last one
      const int r = min(VTW * 16 * w + 16 * i + lrow, rows - 1);
      const uint32_t off = (uint32_t)r * (uint32_t)(2 * K) + (uint32_t)(16 * lchunk) + kb;
      dma16(wbase, off, slot + (uint32_t)(VTW * 16 * w + 16 * i) * RB);
    }
    dma16(a.hidden, hoff + kb, slot + WBW + (uint32_t)(16 * w) * RB);
  };

  // read side: fragment of row (tile base) + l16, chunk g4 at position g4 ^ ((l16 >> 2) & 3)
  const int l16 = lane & 15, g4 = lane >> 4;
  const uint32_t fro = (uint32_t)(l16 * RB + ((g4 ^ ((l16 >> 2) & 3)) << 4));
  f32x4 acc[VTW][MTL];
#pragma unroll
  for (int i = 0; i < VTW; ++i)
#pragma unroll
    for (int j = 0; j < MTL; ++j) acc[i][j] = (f32x4){};

  issue(0);
  if (S > 1) issue(1);
  for (int v = 0; v < S; ++v) {
    // this wave's loads of stage v have landed (stage v + 1's vtv + 1 may not)
    if (v + 1 < S) {
      switch (vtv) {
        case 0: wait_vmcnt<1>(); break;
        case 1: wait_vmcnt<2>(); break;
        case 2: wait_vmcnt<3>(); break;
        case 3: wait_vmcnt<4>(); break;
        case 4: wait_vmcnt<5>(); break;
        default: wait_vmcnt<LPW>(); break;
      }
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();                   // every wave's stage-v loads have landed; slot (v + 2) % 3 is free
    if (v + 2 < S) issue(v + 2);
    const uint8_t* base = smem + (v % NBW) * SBW;
    bf16x8 hf[MTL];
#pragma unroll
    for (int j = 0; j < MTL; ++j) hf[j] = *reinterpret_cast<const bf16x8*>(base + WBW + 16 * j * RB + fro);
#pragma unroll
    for (int i = 0; i < VTW; ++i) {
      if (i >= vtv) break;
      const bf16x8 wf = *reinterpret_cast<const bf16x8*>(base + (VTW * 16 * w + 16 * i) * RB + fro);
#pragma unroll
      for (int j = 0; j < MTL; ++j) acc[i][j] = mfma16(wf, hf[j], acc[i][j]);
    }
  }
  // C register r of accumulator (i, j): weight row 80 w + 16 i + 4 g4 + r of the range, drafted row 16 j + l16
#pragma unroll
  for (int j = 0; j < MTL; ++j) {
    const int m = 16 * j + l16;
    if (m >= a.M) continue;
    uint16_t* orow = a.out + (int64_t)m * a.out_stride + R0;
#pragma unroll
    for (int i = 0; i < VTW; ++i) {
      const int n = VTW * 16 * w + 16 * i + 4 * g4;
      const f32x4 c = acc[i][j];
      const u32x2 pk = {__builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){c[0], c[1]}, bf16x2)),
                        __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){c[2], c[3]}, bf16x2))};
      if (n + 4 <= rows) {
        *reinterpret_cast<u32x2*>(orow + n) = pk;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < rows) orow[n + e] = (uint16_t)(pk[e >> 1] >> (16 * (e & 1)));
      }
    }
  }
}

}  // namespace

static int draft_head_gemm(const uint16_t* hidden, int64_t row_stride, int rows_per_group, int64_t group_stride,
                           const uint16_t* weight, int M, int N, int K, uint16_t* out, int64_t out_stride,
                           void* stream, const char* who) {
  if (!hidden || !weight || !out) return mfd_set_error(MFD_ERR_INVALID_ARG, "%s: null pointer", who);
  if (M < 1 || N < 1 || K < 1 || rows_per_group < 1 || row_stride < 0 || group_stride < 0)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "%s: bad sizes M=%d N=%d K=%d rows_per_group=%d", who, M, N, K,
                         rows_per_group);
  if (K % KS != 0)
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "%s: needs K %% %d == 0 (K=%d)", who, KS, K);
  if (row_stride % 8 != 0 || group_stride % 8 != 0 || out_stride < N || out_stride % 4 != 0 ||
      (reinterpret_cast<uintptr_t>(hidden) & 15) || (reinterpret_cast<uintptr_t>(weight) & 15) ||
      (reinterpret_cast<uintptr_t>(out) & 7))
    return mfd_set_error(MFD_ERR_UNSUPPORTED,
                         "%s: drafted rows and weight need 16-byte alignment, output rows 8-byte alignment "
                         "(row_stride=%lld group_stride=%lld out_stride=%lld)",
                         who, (long long)row_stride, (long long)group_stride, (long long)out_stride);
  // one workgroup per CU (128 KB of LDS each), at least 128 weight rows each
  const int nwg = std::max(1, std::min(mfd_num_cus(), (N + PT - 1) / PT));
  const int64_t maxrows = (int64_t)N / nwg + 8;
  if (maxrows * K * 2 >= ((int64_t)1 << 32) ||
      ((int64_t)(M - 1) / rows_per_group * group_stride + (int64_t)rows_per_group * row_stride + K) * 2 >=
          ((int64_t)1 << 32))
    return mfd_set_error(MFD_ERR_UNSUPPORTED, "%s: N=%d K=%d M=%d too large for 32-bit offsets", who, N, K, M);
  {
    // the kernels' dynamic LDS limits, raised once per device
    int rc = mfd_set_max_lds(reinterpret_cast<const void*>(&draft_head_kernel), SMEM);
    if (rc == MFD_OK) rc = mfd_set_max_lds(reinterpret_cast<const void*>(&draft_head_wide_kernel), wide::SMEMW);
    if (rc != MFD_OK) return rc;
  }
  // workgroup ranges of more than two 128-row passes (and at most wide::WRMAX rows): the wide form, which streams
  // the drafted rows once per workgroup instead of once per pass
  const bool wide_form = maxrows > 2 * PT && maxrows <= wide::WRMAX;
  // one launch per 128 drafted rows (each streams the weight once)
  for (int m0 = 0; m0 < M; m0 += MT) {
    HeadArgs a{hidden, row_stride, group_stride, rows_per_group, m0, weight, out + (int64_t)m0 * out_stride,
               out_stride, std::min(MT, M - m0), N, K, nwg};
    if (wide_form)
      hipLaunchKernelGGL(draft_head_wide_kernel, dim3(nwg), dim3(wide::NTH), wide::SMEMW,
                         static_cast<hipStream_t>(stream), a);
    else
      hipLaunchKernelGGL(draft_head_kernel, dim3(nwg), dim3(NT), SMEM, static_cast<hipStream_t>(stream), a);
    MFD_CHECK_LAUNCH();
  }
  return MFD_OK;
}

extern "C" int mfd_draft_head_gemm(const uint16_t* hidden, int64_t row_stride, int rows_per_group,
                                   int64_t group_stride, const uint16_t* weight, int M, int N, int K, uint16_t* out,
                                   int64_t out_stride, void* stream) {
  return draft_head_gemm(hidden, row_stride, rows_per_group, group_stride, weight, M, N, K, out, out_stride, stream,
                         "mfd_draft_head_gemm");
}

extern "C" int mfd_draft_topk_head(const uint16_t* hidden, int64_t row_stride, int rows_per_group,
                                   int64_t group_stride, const uint16_t* weight, int M, int N, int K,
                                   uint16_t* logits, int64_t logits_stride, int k, float* out_logp, void* out_ids,
                                   int ids_int64, float* out_logz, const int32_t* vocab_ids, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  if (M == 0) return MFD_OK;
  const int rc = draft_head_gemm(hidden, row_stride, rows_per_group, group_stride, weight, M, N, K, logits,
                                 logits_stride, stream, "mfd_draft_topk_head");
  if (rc != MFD_OK) return rc;
  return vocab_ids ? mfd_topk_logz_vocab(logits, M, N, logits_stride, k, out_logp, out_ids, ids_int64, out_logz,
                                         vocab_ids, workspace, workspace_bytes, stream)
                   : mfd_topk_logz(logits, M, N, logits_stride, k, out_logp, out_ids, ids_int64, out_logz, workspace,
                                   workspace_bytes, stream);
}
