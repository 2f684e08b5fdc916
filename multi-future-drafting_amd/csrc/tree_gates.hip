// Gates of a Gated-DeltaNet layer over a draft tree, for gfx950.
//
// Follows inference/hf/qwen35_tree.py:77-79: beta = sigmoid(float(b)),
// g = -exp(float(A_log)) * softplus(float(a) + float(dt_bias)) (torch's softplus: x above 20 is returned
// as is, else log1p(exp(x))), and G = anc @ g, the log decay summed over the node's ancestors and itself.
// The reference forms G with a dense [n, n] x [n, H] product; here each (node, head) thread walks its parent
// pointers and sums g from the root down (parents precede children, so the walk ends at the root).
#include "mfd_common.h"

namespace {

constexpr int MAX_WALK = 4096;  // parent steps before a malformed (cyclic) tree is rejected

struct GatesArgs {
  const void* a;
  const void* b;
  int ab_bf16;
  int64_t ab_st;  // row stride of a and b (elements)
  const float* A_log;
  const float* dt_bias;
  const int32_t* parents;
  const int8_t* anc8;
  const int32_t* cu_nodes;
  int R, N, H;
  float* g_cum;
  float* beta;
  int32_t* err;
};

__device__ __forceinline__ float load_ab(const void* p, int ab_bf16, int64_t idx) {
  return ab_bf16 ? bf2f(reinterpret_cast<const uint16_t*>(p)[idx]) : reinterpret_cast<const float*>(p)[idx];
}

__device__ __forceinline__ float softplus_torch(float x) { return x > 20.f ? x : log1pf(expf(x)); }

__device__ __forceinline__ float gate_g(const GatesArgs& a, int node, int h) {
  const float x = load_ab(a.a, a.ab_bf16, (int64_t)node * a.ab_st + h) + a.dt_bias[h];
  return -expf(a.A_log[h]) * softplus_torch(x);
}

__global__ __launch_bounds__(256) void tree_gates_kernel(GatesArgs a) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)a.N * a.H) return;
  const int node = (int)(t / a.H);
  const int h = (int)(t % a.H);
  // request of this node: cu_nodes is sorted, R is small
  int r = 0, ns = 0;
  if (a.cu_nodes) {
    int lo = 0, hi = a.R - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.cu_nodes[mid] <= node) lo = mid; else hi = mid - 1;
    }
    r = lo;
    ns = a.cu_nodes[r];
  }
  (void)r;
  const int il = node - ns;
  a.beta[t] = 1.f / (1.f + expf(-load_ab(a.b, a.ab_bf16, (int64_t)node * a.ab_st + h)));
  // parent of a request-local node: from the parents array, or the largest strict ancestor in anc8
  auto parent_of = [&](int i) -> int {
    if (a.parents) return a.parents[ns + i];
    const int8_t* row = a.anc8 + (int64_t)i * a.N;
    for (int j = i - 1; j >= 0; --j)
      if (row[j] != 0) return j;
    return -1;
  };
  // depth first, then sum from the root down: the s-th ancestor is found by walking again
  int d = 0;
  for (int cur = il; cur >= 0; ++d) {
    const int p = parent_of(cur);
    if (p >= cur || d >= MAX_WALK) {
      if (a.err) atomicOr(a.err, MFD_DEVERR_NOT_TOPOLOGICAL);
      a.g_cum[t] = __builtin_nanf("");
      return;
    }
    cur = p;
  }
  float G = 0.f;
  for (int s = d - 1; s >= 0; --s) {  // s = steps from the node up to the summed ancestor
    int cur = il;
    for (int x = 0; x < s; ++x) cur = parent_of(cur);
    G += gate_g(a, ns + cur, h);
  }
  a.g_cum[t] = G;
}

}  // namespace

extern "C" int mfd_tree_gates(const void* a_proj, const void* b_proj, int ab_bf16, int64_t ab_row_stride,
                              const float* A_log, const float* dt_bias, const int32_t* parents, const int8_t* anc8,
                              const int32_t* cu_nodes, int R, int N, int H, float* g_cum, float* beta,
                              int32_t* err_flag, void* stream) {
  if (R < 1 || N < 0 || H < 1 || ab_row_stride < H)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gates: bad sizes R=%d N=%d H=%d stride=%lld", R, N, H,
                         (long long)ab_row_stride);
  if (!cu_nodes && R != 1) return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gates: cu_nodes required for R > 1");
  if (!parents && (!anc8 || R != 1))
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gates: parents required unless R == 1 and anc8 given");
  if (N == 0) return MFD_OK;
  if (!a_proj || !b_proj || !A_log || !dt_bias || !g_cum || !beta)
    return mfd_set_error(MFD_ERR_INVALID_ARG, "mfd_tree_gates: null tensor pointer");
  GatesArgs args{a_proj, b_proj, ab_bf16 ? 1 : 0, ab_row_stride, A_log, dt_bias, parents, anc8, cu_nodes, R, N, H,
                 g_cum, beta, err_flag};
  const int64_t total = (int64_t)N * H;
  hipLaunchKernelGGL(tree_gates_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), args);
  MFD_CHECK_LAUNCH();
  return MFD_OK;
}
