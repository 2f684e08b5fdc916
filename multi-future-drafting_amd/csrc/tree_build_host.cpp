// Host (CPU) form of the exact tree builders, for callers whose inputs and outputs live in host memory: the
// SGLang patch's synchronous path calls build_trees with CPU tensors every round (inference/sglang/patches/
// sglang-v0.5.22-mfd.patch:1431-1445, 2889-2897), and the HF builders take and return host tensors
// (inference/hf/tree_build_ext.py:118-234). Same trees, node for node, as the device builders (tree_build.hip)
// and the reference's heaps (P:1256-1407):
//   mixture (K > 1): pop order by (float key -(float(logw) + prior[mode]), mode, parent, depth, rank, logw),
//     smallest first; a popped candidate whose token its parent already has is merged into that child
//   single mode (K = 1): pop order by (fp64 key -logw, rank tuple compared as a Python tuple, parent, depth, rank,
//     logw); every pop is a new node
//   after a pop: the next sibling (rank + 1, logw - lp[rank] + lp[rank + 1]) and the first child (depth + 1,
//     logw + lp[depth][0]) become candidates.
// The frontier is a flat binary heap ordered by that total order (entries that compare equal are identical, so the
// pop sequence does not depend on the heap's layout); children are found through an open-addressing table keyed by
// (parent, token); the rank tuples of the single-mode order are kept per node and compared only on equal keys.
#include <cstdint>
#include <cstring>
#include <vector>

#include "mfd_common.h"

namespace {

struct Cand {
  double key;   // single mode: -logw; mixture: the float key widened (exactly) to double
  double logw;  // without the prior
  int32_t mode, parent, depth, rank;
};

// Per-call state, reused across requests.
struct HostBuilder {
  std::vector<Cand> heap;
  std::vector<int64_t> slot_key;   // (parent << 32) | token, -1 = empty
  std::vector<int32_t> slot_node;
  std::vector<uint16_t> tuples;    // single mode: rank tuple of node i at tuples[i * (L + 1) ..], length depth[i]
  int L = 0;
  bool single = false;
  const int64_t* depth_of = nullptr;  // depths of the nodes built so far (single mode)

  // lexicographic comparison of (tuple of node p) + [r] against (tuple of node q) + [s]: < 0, 0, > 0
  int cmp_tuples(int p, int r, int q, int s) const {
    const int dp = (int)depth_of[p], dq = (int)depth_of[q];
    const uint16_t* tp = &tuples[(size_t)p * (L + 1)];
    const uint16_t* tq = &tuples[(size_t)q * (L + 1)];
    const int n = dp < dq ? dp : dq;
    for (int i = 0; i < n; ++i)
      if (tp[i] != tq[i]) return tp[i] < tq[i] ? -1 : 1;
    // one prefix ends: compare the next element (the entry's own rank, or the longer tuple's element)
    const int a = dp == n ? r : tp[n];
    const int b = dq == n ? s : tq[n];
    if (a != b) return a < b ? -1 : 1;
    if (dp == dq) return 0;
    // equal so far: the shorter of the two full tuples (length depth + 1) is smaller
    return dp < dq ? -1 : 1;
  }

  // true when a pops before b
  bool before(const Cand& a, const Cand& b) const {
    if (a.key != b.key) return a.key < b.key;
    if (single) {
      const int c = cmp_tuples(a.parent, a.rank, b.parent, b.rank);
      if (c != 0) return c < 0;
    } else if (a.mode != b.mode) {
      return a.mode < b.mode;
    }
    if (a.parent != b.parent) return a.parent < b.parent;
    if (a.depth != b.depth) return a.depth < b.depth;
    if (a.rank != b.rank) return a.rank < b.rank;
    return a.logw < b.logw;
  }

  void push(const Cand& c) {
    heap.push_back(c);
    size_t i = heap.size() - 1;
    while (i > 0) {
      const size_t up = (i - 1) / 2;
      if (!before(heap[i], heap[up])) break;
      std::swap(heap[i], heap[up]);
      i = up;
    }
  }
  Cand pop() {
    const Cand top = heap[0];
    heap[0] = heap.back();
    heap.pop_back();
    size_t i = 0;
    const size_t n = heap.size();
    for (;;) {
      const size_t l = 2 * i + 1, r = l + 1;
      size_t m = i;
      if (l < n && before(heap[l], heap[m])) m = l;
      if (r < n && before(heap[r], heap[m])) m = r;
      if (m == i) break;
      std::swap(heap[i], heap[m]);
      i = m;
    }
    return top;
  }

  // child of `parent` with `token`, or -1; insert = the node to record when absent
  int32_t child(int32_t parent, int64_t token, int32_t insert) {
    const int64_t k = ((int64_t)parent << 32) | (uint32_t)token;
    const size_t mask = slot_key.size() - 1;
    size_t h = (size_t)((uint64_t)k * 0x9E3779B97F4A7C15ull >> 20) & mask;
    for (;;) {
      if (slot_key[h] == -1) {
        if (insert >= 0) {
          slot_key[h] = k;
          slot_node[h] = insert;
        }
        return -1;
      }
      if (slot_key[h] == k) return slot_node[h];
      h = (h + 1) & mask;
    }
  }
};

// One request. lp / ids [K, L, k] (ids int32 or int64); prior [K] or NULL. Writes tokens / depths / parents
// [budget + 1]; returns n. single: the DDTree heap (K must be 1).
template <typename Id>
int64_t build_one(HostBuilder& hb, const float* lp, const Id* ids, const float* prior, int K, int L, int k, int budget,
                  bool single, int64_t* tokens, int64_t* depths, int64_t* parents) {
  auto at = [&](int mode, int d, int r) { return ((size_t)mode * L + d) * k + r; };
  auto key_of = [&](double logw, int mode) {
    if (single) return -logw;
    const float pr = prior ? prior[mode] : 0.f;
    return (double)(-((float)logw + pr));
  };
  hb.single = single;
  hb.L = L;
  hb.depth_of = depths;
  hb.heap.clear();
  if (single) {
    hb.tuples.assign((size_t)(budget + 1) * (L + 1), 0);
  } else {
    size_t cap = 16;
    while (cap < (size_t)budget * 2 + 2) cap <<= 1;
    hb.slot_key.assign(cap, -1);
    hb.slot_node.assign(cap, 0);
  }
  tokens[0] = 0;
  depths[0] = 0;
  parents[0] = -1;
  for (int mode = 0; mode < K; ++mode) {
    const double lw = (double)lp[at(mode, 0, 0)];
    hb.push(Cand{key_of(lw, mode), lw, mode, 0, 1, 0});
  }
  int64_t count = 0;
  while (!hb.heap.empty() && count < budget) {
    const Cand e = hb.pop();
    const int64_t token = (int64_t)ids[at(e.mode, e.depth - 1, e.rank)];
    int32_t cur = single ? -1 : hb.child(e.parent, token, -1);
    if (cur < 0) {
      cur = (int32_t)(count + 1);
      tokens[cur] = token;
      depths[cur] = e.depth;
      parents[cur] = e.parent;
      if (single) {
        uint16_t* t = &hb.tuples[(size_t)cur * (L + 1)];
        const uint16_t* tp = &hb.tuples[(size_t)e.parent * (L + 1)];
        for (int i = 0; i + 1 < e.depth; ++i) t[i] = tp[i];
        t[e.depth - 1] = (uint16_t)e.rank;
      } else {
        hb.child(e.parent, token, cur);
      }
      ++count;
    }
    if (e.rank + 1 < k) {
      const double lw = e.logw - (double)lp[at(e.mode, e.depth - 1, e.rank)] + (double)lp[at(e.mode, e.depth - 1, e.rank + 1)];
      hb.push(Cand{key_of(lw, e.mode), lw, e.mode, e.parent, e.depth, e.rank + 1});
    }
    if (e.depth < L) {
      const double lw = e.logw + (double)lp[at(e.mode, e.depth, 0)];
      hb.push(Cand{key_of(lw, e.mode), lw, e.mode, cur, e.depth + 1, 0});
    }
  }
  return count;
}

}  // namespace

extern "C" int mfd_build_trees_host(const float* top_logp, const void* top_ids, int ids_int64, const float* log_prior,
                                    int bs, int K, int L, int k, int budget, int single_mode_heap, int64_t* tree_out,
                                    int64_t* counts_out, int8_t* anc8_out) {
  if (bs < 0 || K < 1 || L < 1 || k < 1 || budget < 0 || K > 65535 || L > 65535 || k > 65535)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_build_trees_host: bad sizes bs=%d K=%d L=%d k=%d budget=%d", bs, K,
                         L, k, budget);
  if (bs == 0) return MFD_OK;
  if (!top_logp || !top_ids || !tree_out || !counts_out)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_build_trees_host: null pointer");
  const int64_t width = (int64_t)budget + 1;
  const size_t per = (size_t)K * L * k;
  const bool single = single_mode_heap != 0 && K == 1;
  HostBuilder hb;
  hb.heap.reserve((size_t)2 * budget + K + 2);
  for (int b = 0; b < bs; ++b) {
    int64_t* t = tree_out + (size_t)b * 3 * width;
    int64_t* d = t + width;
    int64_t* p = d + width;
    const float* pr = log_prior ? log_prior + (size_t)b * K : nullptr;
    const int64_t n = ids_int64
        ? build_one(hb, top_logp + b * per, static_cast<const int64_t*>(top_ids) + b * per, pr, K, L, k, budget, single, t, d, p)
        : build_one(hb, top_logp + b * per, static_cast<const int32_t*>(top_ids) + b * per, pr, K, L, k, budget, single, t, d, p);
    for (int64_t i = n + 1; i < width; ++i) {
      t[i] = 0;
      d[i] = 0;
      p[i] = -1;
    }
    counts_out[b] = n;
    if (anc8_out) {  // ancestor-or-self rows: row i = its parent's row plus column i (parents precede children)
      int8_t* v = anc8_out + (size_t)b * width * width;
      std::memset(v, 0, (size_t)width * width);
      for (int64_t i = 0; i <= n; ++i) {
        int8_t* row = v + (size_t)i * width;
        if (i > 0) std::memcpy(row, v + (size_t)p[i] * width, (size_t)i);
        row[i] = 1;
      }
    }
  }
  return MFD_OK;
}
