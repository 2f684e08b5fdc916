/* CPU oracle, C restatement. TEST INFRASTRUCTURE ONLY (never linked into the product library).
 *
 * 1. Mixture-tree best-first builder (exact node order).
 *    Restates the reference's heap (inference/hf/tree_build_ext.py:48-62 MixEntry/MixGreater,
 *    :158-203 build_mixture; the batched form inference/sglang/patches/sglang-v0.5.22-mfd.patch
 *    :1330-1407): key -(float(logw) + prior[mode]) in float32, logw accumulated in double as
 *    (logw - lp[r]) + lp[r+1] for a sibling and logw + lp[d][0] for a child, ties broken by
 *    (mode, parent, depth, rank, logw) ascending; a prefix popped again by another mode reuses
 *    its node; the budget counts distinct nodes.
 *    Single-mode DDTree (tree_build_ext.py:31-46, :118-156): key -logw in double, ties by the
 *    lexicographic rank tuple, then parent, depth, rank, logw.
 *
 * 2. Logits pass (the product's definition of top-k + log Z, reference semantics
 *    inference/hf/tree_logits.py:34-46 with an explicit, deterministic reduction):
 *    - top-k by value descending, ties by token id ascending;
 *    - log Z over pieces of MFD_LZ_CHUNK = 2048 elements: piece max m_c; element 512 j + 8 l + e of the
 *      piece belongs to lane l (l < 64, j < 4, e < 8), which sums its elements in (j, e) order from 0:
 *      s = fmaf(E(x), E(-m_c), s) when -60 <= m_c < 64, with E the float table of e^x over the bf16 values
 *      2^-25 <= |x| < 128 (index min(max(rotl16(bits, 1) - 0x6600, 0), 8191)), else
 *      s = s + exp_det(max(x - m_c, -80)) (nothing for an all -inf piece); the 64 lane sums are added
 *      pairwise over lane distances 32, 16, 8, 4, 2, 1 into S_c (float);
 *      Z = sum_c S_c * exp_det(max(m_c - m, -80)) in double in piece order; log Z = float(m + log_det(Z)).
 *    exp_det / log_det use only IEEE +, *, fma, division and exact power-of-two scaling, and the table entries
 *    are e^x in double rounded to float, so the HIP kernel computing the same sequence (with the same table,
 *    exp_bf16_table.h, generated the same way) gets the same bits.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define MFD_LZ_CHUNK 2048

/* ------------------------------------------------------------------ deterministic math */

static float pow2i(int k) { /* exact 2^k for -126 <= k <= 127 */
  uint32_t bits = (uint32_t)(k + 127) << 23;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

float oracle_exp_det(float d) { /* e^d for d in [-80, 0] */
  float k = rintf(d * 1.44269504088896341f);
  float r = fmaf(k, -0.693145751953125f, d);
  r = fmaf(k, -1.42860676533018592e-06f, r);
  float p = 2.48015873015873016e-05f;   /* 1/8! */
  p = fmaf(p, r, 1.98412698412698413e-04f); /* 1/7! */
  p = fmaf(p, r, 1.38888888888888889e-03f); /* 1/6! */
  p = fmaf(p, r, 8.33333333333333333e-03f); /* 1/5! */
  p = fmaf(p, r, 4.16666666666666667e-02f); /* 1/4! */
  p = fmaf(p, r, 1.66666666666666667e-01f); /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return p * pow2i((int)k);
}

double oracle_log_det(double z) { /* natural log for z >= 1 (finite) */
  int e;
  double f = frexp(z, &e); /* z = f 2^e, f in [0.5, 1) */
  if (f < 0.70710678118654752440) {
    f = f * 2.0;
    e -= 1;
  }
  double s = (f - 1.0) / (f + 1.0);
  double s2 = s * s;
  /* 2 atanh(s) = 2 (s + s^3/3 + ... + s^23/23) */
  double p = 1.0 / 23.0;
  p = fma(p, s2, 1.0 / 21.0);
  p = fma(p, s2, 1.0 / 19.0);
  p = fma(p, s2, 1.0 / 17.0);
  p = fma(p, s2, 1.0 / 15.0);
  p = fma(p, s2, 1.0 / 13.0);
  p = fma(p, s2, 1.0 / 11.0);
  p = fma(p, s2, 1.0 / 9.0);
  p = fma(p, s2, 1.0 / 7.0);
  p = fma(p, s2, 1.0 / 5.0);
  p = fma(p, s2, 1.0 / 3.0);
  p = fma(p, s2, 1.0);
  double logf_ = 2.0 * s * p;
  double de = (double)e;
  return fma(de, 6.93147180369123816490e-01, fma(de, 1.90821492927058770002e-10, logf_));
}

static float bf16_to_f32(uint16_t b) {
  uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* e^x rounded to float for the bf16 values x with 2^-25 <= |x| < 128; entry i belongs to the bit pattern
   whose rotl16 by 1 is i + 0x6600 (magnitude bits 0x3300 + i / 2, sign i % 2) */
#define EXP_TAB 8192
static float exp_tab[EXP_TAB];
static int exp_tab_ready = 0;
static void exp_tab_init(void) {
  if (exp_tab_ready) return;
  for (int i = 0; i < EXP_TAB; ++i) {
    uint32_t r = (uint32_t)i + 0x6600u;
    uint16_t b = (uint16_t)((r >> 1) | ((r & 1u) << 15));
    exp_tab[i] = (float)exp((double)bf16_to_f32(b));
  }
  exp_tab_ready = 1;
}
static int exp_tab_index(uint16_t b) {
  int r = (int)((((uint32_t)b << 1) | ((uint32_t)b >> 15)) & 0xFFFFu) - 0x6600;
  return r < 0 ? 0 : (r > EXP_TAB - 1 ? EXP_TAB - 1 : r);
}
float oracle_exp_table(int i) {
  exp_tab_init();
  return exp_tab[i & (EXP_TAB - 1)];
}

static uint16_t f32_to_bf16_bits(float f) { /* f is a widened bf16 value: its upper half */
  uint32_t bits;
  memcpy(&bits, &f, 4);
  return (uint16_t)(bits >> 16);
}

/* S_c of one piece of n <= MFD_LZ_CHUNK valid elements with maximum m (the lane order above) */
float oracle_chunk_sum(const uint16_t* x, int n, float m) {
  exp_tab_init();
  float v[64], u[64];
  const int fast = m >= -60.0f && m < 64.0f;
  const float C = fast ? exp_tab[exp_tab_index((uint16_t)(f32_to_bf16_bits(m) ^ 0x8000u))] : 0.0f;
  for (int l = 0; l < 64; ++l) {
    float s = 0.0f;
    for (int j = 0; j < 4; ++j)
      for (int e = 0; e < 8; ++e) {
        int i = 512 * j + 8 * l + e;
        if (fast) {
          uint16_t b = i < n ? x[i] : (uint16_t)0xFF80u; /* past the row end: -inf, table entry 0.0 */
          s = fmaf(exp_tab[exp_tab_index(b)], C, s);
        } else if (m != -INFINITY) {
          float term = 0.0f;
          if (i < n) {
            float d = bf16_to_f32(x[i]) - m;
            d = d > -80.0f ? d : -80.0f;
            term = oracle_exp_det(d);
          }
          s = s + term;
        }
      }
    v[l] = s;
  }
  for (int d = 32; d >= 1; d >>= 1) {
    for (int l = 0; l < 64; ++l) u[l] = v[l] + v[l ^ d];
    memcpy(v, u, sizeof v);
  }
  return v[0];
}

float oracle_logz_row(const uint16_t* row, int64_t V) {
  int64_t nchunks = (V + MFD_LZ_CHUNK - 1) / MFD_LZ_CHUNK;
  float* mc = (float*)malloc(sizeof(float) * (size_t)(nchunks > 0 ? nchunks : 1));
  double* sc = (double*)malloc(sizeof(double) * (size_t)(nchunks > 0 ? nchunks : 1));
  float m = -INFINITY;
  for (int64_t c = 0; c < nchunks; ++c) {
    int64_t a = c * MFD_LZ_CHUNK, b = a + MFD_LZ_CHUNK < V ? a + MFD_LZ_CHUNK : V;
    float mx = -INFINITY;
    for (int64_t i = a; i < b; ++i) {
      float x = bf16_to_f32(row[i]);
      if (x > mx) mx = x;
    }
    mc[c] = mx;
    sc[c] = (double)oracle_chunk_sum(row + a, (int)(b - a), mx);
    if (mx > m) m = mx;
  }
  float out;
  if (m == -INFINITY) {
    out = -INFINITY;
  } else {
    double z = 0.0;
    for (int64_t c = 0; c < nchunks; ++c) {
      if (mc[c] == -INFINITY) continue;
      float d = mc[c] - m;
      d = d > -80.0f ? d : -80.0f;
      z += sc[c] * (double)oracle_exp_det(d);
    }
    out = (float)((double)m + oracle_log_det(z));
  }
  free(mc);
  free(sc);
  return out;
}

/* top-k of one bf16 row: value descending, token id ascending; k <= V */
void oracle_topk_row(const uint16_t* row, int64_t V, int k, float* vals, int64_t* ids) {
  for (int j = 0; j < k; ++j) { vals[j] = -INFINITY; ids[j] = INT64_MAX; }
  int filled = 0;
  for (int64_t i = 0; i < V; ++i) {
    float x = bf16_to_f32(row[i]);
    if (filled == k && !(x > vals[k - 1])) continue; /* equal value: the earlier id stays */
    int pos = filled < k ? filled : k - 1;
    while (pos > 0 && x > vals[pos - 1]) {
      vals[pos] = vals[pos - 1];
      ids[pos] = ids[pos - 1];
      --pos;
    }
    vals[pos] = x;
    ids[pos] = i;
    if (filled < k) ++filled;
  }
}

/* logits [rows, V] bf16 -> top log-probs [rows, k] f32 (value - logZ in float32) and ids */
void oracle_top_candidates(const uint16_t* logits, int64_t rows, int64_t V, int k, float* logp, int64_t* ids,
                           float* logz_out) {
  float* vals = (float*)malloc(sizeof(float) * (size_t)k);
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* row = logits + r * V;
    float lz = oracle_logz_row(row, V);
    oracle_topk_row(row, V, k, vals, ids + r * k);
    for (int j = 0; j < k; ++j) logp[r * k + j] = vals[j] - lz;
    if (logz_out) logz_out[r] = lz;
  }
  free(vals);
}

/* ------------------------------------------------------------------ mixture heap */

typedef struct {
  float key;
  int mode, parent, depth, rank;
  double logw;
} MixEntry;

/* a pops before b */
static int mix_less(const MixEntry* a, const MixEntry* b) {
  if (a->key != b->key) return a->key < b->key;
  if (a->mode != b->mode) return a->mode < b->mode;
  if (a->parent != b->parent) return a->parent < b->parent;
  if (a->depth != b->depth) return a->depth < b->depth;
  if (a->rank != b->rank) return a->rank < b->rank;
  return a->logw < b->logw;
}

typedef struct {
  MixEntry* a;
  int64_t n, cap;
} MixHeap;

static void mh_push(MixHeap* h, MixEntry e) {
  if (h->n == h->cap) {
    h->cap = h->cap ? 2 * h->cap : 64;
    h->a = (MixEntry*)realloc(h->a, sizeof(MixEntry) * (size_t)h->cap);
  }
  int64_t i = h->n++;
  while (i > 0) {
    int64_t p = (i - 1) / 2;
    if (!mix_less(&e, &h->a[p])) break;
    h->a[i] = h->a[p];
    i = p;
  }
  h->a[i] = e;
}

static MixEntry mh_pop(MixHeap* h) {
  MixEntry top = h->a[0];
  MixEntry last = h->a[--h->n];
  int64_t i = 0;
  for (;;) {
    int64_t c = 2 * i + 1;
    if (c >= h->n) break;
    if (c + 1 < h->n && mix_less(&h->a[c + 1], &h->a[c])) ++c;
    if (!mix_less(&h->a[c], &last)) break;
    h->a[i] = h->a[c];
    i = c;
  }
  if (h->n > 0) h->a[i] = last;
  return top;
}

/* (parent, token) -> node hash, open addressing */
typedef struct {
  int64_t* keys_parent;
  int64_t* keys_token;
  int64_t* vals;
  int64_t cap;
} ChildMap;

static void cm_init(ChildMap* m, int64_t budget) {
  int64_t cap = 16;
  while (cap < 4 * (budget + 1)) cap *= 2;
  m->cap = cap;
  m->keys_parent = (int64_t*)malloc(sizeof(int64_t) * (size_t)cap);
  m->keys_token = (int64_t*)malloc(sizeof(int64_t) * (size_t)cap);
  m->vals = (int64_t*)malloc(sizeof(int64_t) * (size_t)cap);
  for (int64_t i = 0; i < cap; ++i) m->keys_parent[i] = -1;
}
static void cm_free(ChildMap* m) {
  free(m->keys_parent);
  free(m->keys_token);
  free(m->vals);
}
static uint64_t cm_hash(int64_t p, int64_t t) {
  uint64_t x = (uint64_t)p * 0x9E3779B97F4A7C15ull ^ ((uint64_t)t + 0x632BE59BD9B4E019ull);
  x ^= x >> 29;
  x *= 0xBF58476D1CE4E5B9ull;
  x ^= x >> 32;
  return x;
}
static int64_t cm_find(const ChildMap* m, int64_t p, int64_t t) {
  uint64_t i = cm_hash(p, t) & (uint64_t)(m->cap - 1);
  for (;;) {
    if (m->keys_parent[i] == -1) return -1;
    if (m->keys_parent[i] == p && m->keys_token[i] == t) return m->vals[i];
    i = (i + 1) & (uint64_t)(m->cap - 1);
  }
}
static void cm_put(ChildMap* m, int64_t p, int64_t t, int64_t v) {
  uint64_t i = cm_hash(p, t) & (uint64_t)(m->cap - 1);
  while (m->keys_parent[i] != -1) i = (i + 1) & (uint64_t)(m->cap - 1);
  m->keys_parent[i] = p;
  m->keys_token[i] = t;
  m->vals[i] = v;
}

/* One mixture tree. lp [K, L, k] f32, ids [K, L, k] i64, prior [K] f32. Writes tokens/depths/parents
 * [budget + 1] (index 0 = root: token 0, depth 0, parent -1; tail: 0, 0, -1). Returns the node count.
 * Also returns the number of pops through *pops_out (may be NULL). */
int64_t oracle_build_mixture(const float* lp, const int64_t* ids, const float* prior, int K, int L, int k,
                             int64_t budget, int64_t* tokens, int64_t* depths, int64_t* parents, int64_t* pops_out) {
  int64_t width = budget + 1;
  for (int64_t i = 0; i < width; ++i) { tokens[i] = 0; depths[i] = 0; parents[i] = -1; }
  if (budget <= 0 || L <= 0 || K <= 0 || k <= 0) {
    if (pops_out) *pops_out = 0;
    return 0;
  }
#define AT(m, d, r) (((int64_t)(m) * L + (d)) * k + (r))
  MixHeap h = {0, 0, 0};
  for (int m = 0; m < K; ++m) {
    double lw = (double)lp[AT(m, 0, 0)];
    MixEntry e = {-((float)lw + prior[m]), m, 0, 1, 0, lw};
    mh_push(&h, e);
  }
  ChildMap cm;
  cm_init(&cm, budget);
  int64_t count = 0, pops = 0;
  while (h.n > 0 && count < budget) {
    MixEntry e = mh_pop(&h);
    ++pops;
    int64_t token = ids[AT(e.mode, e.depth - 1, e.rank)];
    int64_t current = cm_find(&cm, e.parent, token);
    if (current < 0) {
      current = count + 1;
      tokens[current] = token;
      depths[current] = e.depth;
      parents[current] = e.parent;
      cm_put(&cm, e.parent, token, current);
      ++count;
    }
    if (e.rank + 1 < k) {
      double lw = e.logw - (double)lp[AT(e.mode, e.depth - 1, e.rank)] + (double)lp[AT(e.mode, e.depth - 1, e.rank + 1)];
      MixEntry s = {-((float)lw + prior[e.mode]), e.mode, e.parent, e.depth, e.rank + 1, lw};
      mh_push(&h, s);
    }
    if (e.depth < L) {
      double lw = e.logw + (double)lp[AT(e.mode, e.depth, 0)];
      MixEntry c = {-((float)lw + prior[e.mode]), e.mode, (int)current, e.depth + 1, 0, lw};
      mh_push(&h, c);
    }
  }
#undef AT
  free(h.a);
  cm_free(&cm);
  if (pops_out) *pops_out = pops;
  return count;
}

/* ------------------------------------------------------------------ single-mode DDTree heap */

#define SINGLE_MAXD 64
typedef struct {
  double key;
  int nranks;
  int ranks[SINGLE_MAXD];
  int parent, depth, rank;
  double logw;
} SingleEntry;

static int ranks_cmp(const SingleEntry* a, const SingleEntry* b) { /* Python tuple order */
  int n = a->nranks < b->nranks ? a->nranks : b->nranks;
  for (int i = 0; i < n; ++i)
    if (a->ranks[i] != b->ranks[i]) return a->ranks[i] < b->ranks[i] ? -1 : 1;
  if (a->nranks != b->nranks) return a->nranks < b->nranks ? -1 : 1;
  return 0;
}
static int single_less(const SingleEntry* a, const SingleEntry* b) {
  if (a->key != b->key) return a->key < b->key;
  int c = ranks_cmp(a, b);
  if (c != 0) return c < 0;
  if (a->parent != b->parent) return a->parent < b->parent;
  if (a->depth != b->depth) return a->depth < b->depth;
  if (a->rank != b->rank) return a->rank < b->rank;
  return a->logw < b->logw;
}

/* One DDTree. lp [L, k] f32, ids [L, k] i64. Same output convention as oracle_build_mixture.
 * Returns -1 if a path is deeper than SINGLE_MAXD. */
int64_t oracle_build_single(const float* lp, const int64_t* ids, int L, int k, int64_t budget, int64_t* tokens,
                            int64_t* depths, int64_t* parents) {
  int64_t width = budget + 1;
  for (int64_t i = 0; i < width; ++i) { tokens[i] = 0; depths[i] = 0; parents[i] = -1; }
  if (budget <= 0 || L <= 0 || k <= 0) return 0;
  if (L > SINGLE_MAXD) return -1;
  int64_t cap = 2 * budget + 8, n = 0;
  SingleEntry* heap = (SingleEntry*)malloc(sizeof(SingleEntry) * (size_t)cap);
#define SPUSH(E)                                                   \
  do {                                                             \
    SingleEntry _e = (E);                                          \
    int64_t _i = n++;                                              \
    while (_i > 0) {                                               \
      int64_t _p = (_i - 1) / 2;                                   \
      if (!single_less(&_e, &heap[_p])) break;                     \
      heap[_i] = heap[_p];                                         \
      _i = _p;                                                     \
    }                                                              \
    heap[_i] = _e;                                                 \
  } while (0)
  SingleEntry first;
  memset(&first, 0, sizeof(first));
  first.logw = (double)lp[0];
  first.key = -first.logw;
  first.nranks = 1;
  first.ranks[0] = 0;
  first.parent = 0;
  first.depth = 1;
  first.rank = 0;
  SPUSH(first);
  int64_t count = 0;
  while (n > 0 && count < budget) {
    SingleEntry e = heap[0];
    SingleEntry last = heap[--n];
    int64_t i = 0;
    for (;;) {
      int64_t c = 2 * i + 1;
      if (c >= n) break;
      if (c + 1 < n && single_less(&heap[c + 1], &heap[c])) ++c;
      if (!single_less(&heap[c], &last)) break;
      heap[i] = heap[c];
      i = c;
    }
    if (n > 0) heap[i] = last;
    int64_t token = ids[(int64_t)(e.depth - 1) * k + e.rank];
    int64_t current = count + 1;
    tokens[current] = token;
    depths[current] = e.depth;
    parents[current] = e.parent;
    ++count;
    if (e.rank + 1 < k) {
      SingleEntry s = e;
      s.ranks[s.nranks - 1] = e.rank + 1;
      s.logw = e.logw - (double)lp[(int64_t)(e.depth - 1) * k + e.rank] + (double)lp[(int64_t)(e.depth - 1) * k + e.rank + 1];
      s.key = -s.logw;
      s.rank = e.rank + 1;
      SPUSH(s);
    }
    if (e.depth < L) {
      SingleEntry c = e;
      c.ranks[c.nranks++] = 0;
      c.logw = e.logw + (double)lp[(int64_t)e.depth * k];
      c.key = -c.logw;
      c.parent = (int)current;
      c.depth = e.depth + 1;
      c.rank = 0;
      SPUSH(c);
    }
  }
#undef SPUSH
  free(heap);
  return count;
}

/* visibility [n+1, n+1] (uint8) from parents[0..n] (tree_build_ext.py:101-110) */
void oracle_visibility(const int64_t* parents, int64_t n, uint8_t* vis) {
  int64_t m = n + 1;
  memset(vis, 0, (size_t)(m * m));
  vis[0] = 1;
  for (int64_t i = 1; i < m; ++i) {
    int64_t p = parents[i];
    memcpy(vis + i * m, vis + p * m, (size_t)i);
    vis[i * m + i] = 1;
  }
}
