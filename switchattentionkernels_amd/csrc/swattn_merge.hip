// Pieces for running the routed prefill over split key ranges (context
// parallelism, ring passes): per-row key bounds of a query shard against a
// KV chunk, and the log2-LSE-weighted merge of the partial results.  gfx950.
//
// Reference tags: V = swiattn_gqa_prefill_varlen.py, F = swiattn_gqa_prefill.py.
// The reference runs one device over the whole key range; it exports LSE in
// the log2 convention (V:15, V:236-241) and splits query and key positions in
// its metadata (V:139-141, V:179-182), which is what these pieces build on.

#include <math.h>

#include <string>

#include "common.h"

namespace swattn {
namespace {

// Query row r sits at global position pos[r] of one causal sequence.  Its
// legal keys are [0, pos] (full) or [pos - window + 1, pos] (local) (F:145-155),
// cut to the chunk [kv_start, kv_end) and given in chunk coordinates; an
// empty cut is start == end.
__global__ __launch_bounds__(256) void shard_bounds_kernel(
    const int32_t* __restrict__ pos, int64_t n, int64_t kv_start, int64_t kv_end, int window,
    int32_t* __restrict__ full_starts, int32_t* __restrict__ local_starts,
    int32_t* __restrict__ causal_ends) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int64_t p = pos[r];
  const int64_t len = kv_end - kv_start;
  auto clip = [&](int64_t g) {   // global key -> chunk coordinate in [0, len]
    const int64_t c = g - kv_start;
    return c < 0 ? 0 : (c > len ? len : c);
  };
  const int64_t end = clip(p + 1);
  const int64_t fs = clip(0);
  const int64_t ls = clip(p - window + 1);
  causal_ends[r] = static_cast<int32_t>(end);
  full_starts[r] = static_cast<int32_t>(fs < end ? fs : end);
  local_starts[r] = static_cast<int32_t>(ls < end ? ls : end);
}

constexpr int kMaxParts = 16;
constexpr int kD = 128;

struct MergeArgs {
  const uint16_t* o[kMaxParts];   // bf16 [rows, 128] per part
  const float* lse[kMaxParts];    // fp32 [rows] per part, log2 convention
  int parts;
};

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// One row of 128 values per 16 lanes (8 values per lane).  For every row:
// M = max over parts of LSE_i (parts at -inf, i.e. with no legal key, carry
// no weight), w_i = 2^(LSE_i - M), LSE = M + log2(sum w_i) and
// O = sum w_i O_i / sum w_i.  A row whose parts are all empty stays empty:
// O = NaN, LSE = -inf, as the attention kernel writes for such a row.
__global__ __launch_bounds__(256) void merge_kernel(const MergeArgs a, uint16_t* __restrict__ out,
                                                    float* __restrict__ lse_out, int64_t rows) {
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 4;
  const int sub = threadIdx.x & 15;
  if (row >= rows) return;
  float m = -INFINITY;
  for (int i = 0; i < a.parts; ++i) m = fmaxf(m, a.lse[i][row]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (m != -INFINITY) {
    for (int i = 0; i < a.parts; ++i) {
      const float li = a.lse[i][row];
      if (li == -INFINITY) continue;
      const float w = exp2f(li - m);
      wsum += w;
      const uint4 v = *reinterpret_cast<const uint4*>(a.o[i] + row * kD + 8 * sub);
      const uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += w * bf16_to_f32(x[e] & 0xffffu);
        acc[2 * e + 1] += w * bf16_to_f32(x[e] >> 16);
      }
    }
  }
  const float inv = 1.0f / wsum;   // 1/0 = inf: an all-empty row becomes 0*inf = NaN
  uint32_t y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    y[e] = f32_to_bf16(acc[2 * e] * inv) | (f32_to_bf16(acc[2 * e + 1] * inv) << 16);
  *reinterpret_cast<uint4*>(out + row * kD + 8 * sub) = make_uint4(y[0], y[1], y[2], y[3]);
  if (sub == 0) lse_out[row] = m == -INFINITY ? -INFINITY : m + log2f(wsum);
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace
}  // namespace swattn

using namespace swattn;

extern "C" {

int swattn_shard_bounds(const int32_t* q_positions, int64_t n_q, int64_t kv_start, int64_t kv_end,
                        int32_t window, int32_t* full_starts, int32_t* local_starts,
                        int32_t* causal_ends, void* stream) {
  if (n_q < 0 || n_q > INT32_MAX || kv_start < 0 || kv_end < kv_start ||
      kv_end - kv_start > INT32_MAX)
    return invalid("swattn_shard_bounds: bad sizes");
  if (window <= 0) return invalid("swattn_shard_bounds: window must be positive");
  if (n_q > 0 && (q_positions == nullptr || full_starts == nullptr || local_starts == nullptr ||
                  causal_ends == nullptr))
    return invalid("swattn_shard_bounds: null pointer");
  if (n_q == 0) return SWATTN_OK;
  hipLaunchKernelGGL(shard_bounds_kernel, dim3(static_cast<uint32_t>(ceil_div(n_q, 256))),
                     dim3(256), 0, as_stream(stream), q_positions, n_q, kv_start, kv_end, window,
                     full_starts, local_starts, causal_ends);
  return launch_status("swattn_shard_bounds");
}

int swattn_merge_partials(const void* const* o_parts, const float* const* lse_parts,
                          int32_t n_parts, void* out, float* lse_out, int64_t rows,
                          int32_t head_dim, void* stream) {
  if (head_dim != kD) return invalid("swattn_merge_partials: head_dim must be 128");
  if (n_parts < 1 || n_parts > kMaxParts)
    return invalid("swattn_merge_partials: n_parts must be in [1, 16]");
  if (rows < 0 || rows > (static_cast<int64_t>(1) << 40))
    return invalid("swattn_merge_partials: bad row count");
  if (rows == 0) return SWATTN_OK;
  if (o_parts == nullptr || lse_parts == nullptr || out == nullptr || lse_out == nullptr)
    return invalid("swattn_merge_partials: null pointer");
  MergeArgs a{};
  for (int i = 0; i < n_parts; ++i) {
    if (o_parts[i] == nullptr || lse_parts[i] == nullptr)
      return invalid("swattn_merge_partials: null part");
    if (!aligned16(o_parts[i]))
      return invalid("swattn_merge_partials: partial outputs and out must be 16-byte aligned");
    a.o[i] = static_cast<const uint16_t*>(o_parts[i]);
    a.lse[i] = lse_parts[i];
  }
  a.parts = n_parts;
  if (!aligned16(out))
    return invalid("swattn_merge_partials: partial outputs and out must be 16-byte aligned");
  const int64_t blocks = ceil_div(rows * 16, 256);
  if (blocks > INT32_MAX) return invalid("swattn_merge_partials: too many rows");
  hipLaunchKernelGGL(merge_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     as_stream(stream), a, static_cast<uint16_t*>(out), lse_out, rows);
  return launch_status("swattn_merge_partials");
}

}  // extern "C"
