// Integer kernels of the routed prefill: router-mask compaction, index-list
// validation and varlen position metadata.  gfx950, wave64.
//
// Reference tags: V = swiattn_gqa_prefill_varlen.py, F = swiattn_gqa_prefill.py.

#include <limits.h>

#include <string>

#include "common.h"

namespace swattn {

static thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }

namespace {

// ---------------------------------------------------------------------------
// Compaction (V:306-322).
//
// A block of 16 waves owns 16384 consecutive mask bytes; wave w owns 16 groups
// of 64 bytes.  Lane l of group e reads byte base + 64e + l, so each group is
// one coalesced 64-byte read and one 64-bit ballot.  popcount(ballot) gives the
// group's full count and mbcnt(ballot) a lane's rank inside the group; the
// ballots stay in scalar registers between the counting pass and the write
// pass, so the mask is read once per kernel.  Full position i lands at
// index excl(i) and local position i at nf + i - excl(i), where excl(i) is the
// number of full positions before i: both lists come out ascending and the
// whole output is exactly arange(n)[mask] ++ arange(n)[~mask].
// ---------------------------------------------------------------------------
constexpr int kCompactWaves = 16;
constexpr int kCompactThreads = kCompactWaves * 64;
constexpr int kCompactGroups = 16;
constexpr int kCompactChunk = kCompactThreads * kCompactGroups;  // 16384 bytes per block

// What decides "full" for position i: a byte mask, or router logits above a
// threshold (compared in fp32; bf16 and fp16 convert exactly, NaN is never
// above the threshold).
struct MaskSource {
  const uint8_t* p;
  __device__ __forceinline__ bool operator()(int64_t i) const { return p[i] != 0; }
};
struct F32LogitSource {
  const float* p;
  float thr;
  __device__ __forceinline__ bool operator()(int64_t i) const { return p[i] > thr; }
};
struct BF16LogitSource {
  const uint16_t* p;
  float thr;
  __device__ __forceinline__ bool operator()(int64_t i) const {
    return __uint_as_float(static_cast<uint32_t>(p[i]) << 16) > thr;
  }
};
struct F16LogitSource {
  const _Float16* p;
  float thr;
  __device__ __forceinline__ bool operator()(int64_t i) const {
    return static_cast<float>(p[i]) > thr;
  }
};

__device__ __forceinline__ int64_t compact_elem(int wave, int e, int lane) {
  return static_cast<int64_t>(blockIdx.x) * kCompactChunk +
         static_cast<int64_t>(wave) * (64 * kCompactGroups) + 64 * e + lane;
}

template <typename Src>
__global__ __launch_bounds__(kCompactThreads) void compact_count_kernel(
    const Src src, int64_t n, int32_t* __restrict__ block_counts) {
  __shared__ int s_wave[kCompactWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int cnt = 0;
#pragma unroll
  for (int e = 0; e < kCompactGroups; ++e) {
    const int64_t i = compact_elem(wave, e, lane);
    const bool f = i < n && src(i);
    cnt += __builtin_popcountll(wave_ballot(f));
  }
  if (lane == 0) s_wave[wave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    int tot = 0;
    for (int w = 0; w < kCompactWaves; ++w) tot += s_wave[w];
    block_counts[blockIdx.x] = tot;
  }
}

// block_counts == nullptr: a single block covers the whole mask.
template <typename Src>
__global__ __launch_bounds__(kCompactThreads) void compact_scatter_kernel(
    const Src src, int64_t n, const int32_t* __restrict__ block_counts,
    int nblocks, int32_t* __restrict__ indices, int32_t* __restrict__ counts) {
  __shared__ int s_wave[kCompactWaves];
  __shared__ int s_prefix, s_total;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t bal[kCompactGroups];
  int cnt = 0;
#pragma unroll
  for (int e = 0; e < kCompactGroups; ++e) {
    const int64_t i = compact_elem(wave, e, lane);
    const bool f = i < n && src(i);
    bal[e] = wave_ballot(f);
    cnt += __builtin_popcountll(bal[e]);
  }
  if (lane == 0) s_wave[wave] = cnt;
  if (wave == 0) {
    int pre = 0, tot = 0;
    if (block_counts != nullptr) {
      for (int j = lane; j < nblocks; j += 64) {
        const int c = block_counts[j];
        tot += c;
        pre += (j < static_cast<int>(blockIdx.x)) ? c : 0;
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        pre += __shfl_xor(pre, off);
        tot += __shfl_xor(tot, off);
      }
    }
    if (lane == 0) {
      s_prefix = pre;
      s_total = tot;
    }
  }
  __syncthreads();
  int wave_prefix = s_prefix, block_total = 0;
  for (int w = 0; w < kCompactWaves; ++w) {
    const int c = s_wave[w];
    wave_prefix += (w < wave) ? c : 0;
    block_total += c;
  }
  const int64_t nf = (block_counts != nullptr) ? s_total : block_total;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    counts[0] = static_cast<int32_t>(nf);
    counts[1] = static_cast<int32_t>(n - nf);
  }
  int64_t full_before = wave_prefix;
#pragma unroll
  for (int e = 0; e < kCompactGroups; ++e) {
    const int64_t i = compact_elem(wave, e, lane);
    const uint64_t b = bal[e];
    const int64_t fb = full_before + count_below(b);
    if (i < n) {
      if ((b >> lane) & 1ull)
        indices[fb] = static_cast<int32_t>(i);
      else
        indices[nf + (i - fb)] = static_cast<int32_t>(i);
    }
    full_before += __builtin_popcountll(b);
  }
}

// ---------------------------------------------------------------------------
// Index validation (V:299-302 on both lists, disjointness of V:341-342).
// One thread per slot; a slot checks its full entry (range, order against the
// previous entry, binary search in the local list) and its local entry (range,
// order).  Any failure ORs its bit into *flags, which flags_clear_kernel zeroes
// first.  The binary search is only meaningful when the local list is sorted;
// when it is not, ERR_LOCAL_ORDER is raised and the caller reports that first.
// ---------------------------------------------------------------------------
__global__ void flags_clear_kernel(int32_t* flags) { flags[0] = 0; }

__global__ __launch_bounds__(256) void check_indices_kernel(
    const int32_t* __restrict__ full, int64_t nf, const int32_t* __restrict__ local, int64_t nl,
    int64_t seq_len, int32_t* __restrict__ flags) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  int f = 0;
  if (i < nf) {
    const int32_t x = full[i];
    if (x < 0 || x >= seq_len) f |= SWATTN_ERR_FULL_RANGE;
    if (i > 0 && x <= full[i - 1]) f |= SWATTN_ERR_FULL_ORDER;
    int64_t lo = 0, hi = nl;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (local[mid] < x)
        lo = mid + 1;
      else
        hi = mid;
    }
    if (lo < nl && local[lo] == x) f |= SWATTN_ERR_OVERLAP;
  }
  if (i < nl) {
    const int32_t x = local[i];
    if (x < 0 || x >= seq_len) f |= SWATTN_ERR_LOCAL_RANGE;
    if (i > 0 && x <= local[i - 1]) f |= SWATTN_ERR_LOCAL_ORDER;
  }
  // One atomic per wave that saw a failure.
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) f |= __shfl_xor(f, off);
  if (f != 0 && (threadIdx.x & 63) == 0) atomicOr(flags, f);
}

// ---------------------------------------------------------------------------
// Varlen metadata (the fields V validates at V:360-383; F's rule per segment).
// One thread per token; the segment is found by binary search in cu_seqlens.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int find_segment(const int32_t* cu, int nseq, int64_t t) {
  int lo = 0, hi = nseq;  // invariant: cu[lo] <= t < cu[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cu[mid] <= t)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(256) void metadata_kernel(
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_kv, int nseq, int64_t total_q,
    int64_t total_kv, int window, int32_t* __restrict__ q_pos, int32_t* __restrict__ kv_pos,
    int32_t* __restrict__ q_seg, int32_t* __restrict__ kv_seg, int32_t* __restrict__ full_starts,
    int32_t* __restrict__ local_starts, int32_t* __restrict__ causal_ends) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < total_q) {
    const int s = find_segment(cu_q, nseq, t);
    const int64_t i = t - cu_q[s];
    const int64_t ks = cu_kv[s], klen = static_cast<int64_t>(cu_kv[s + 1]) - ks;
    q_pos[t] = static_cast<int32_t>(i);
    q_seg[t] = s;
    full_starts[t] = static_cast<int32_t>(ks);
    const int64_t lo = i - window + 1;
    local_starts[t] = static_cast<int32_t>(ks + (lo > 0 ? lo : 0));
    causal_ends[t] = static_cast<int32_t>(ks + (i + 1 < klen ? i + 1 : klen));
  }
  if (t < total_kv) {
    const int s = find_segment(cu_kv, nseq, t);
    kv_pos[t] = static_cast<int32_t>(t - cu_kv[s]);
    kv_seg[t] = s;
  }
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <typename Src>
int compact_impl(const Src& src, bool src_null, int64_t n, int32_t* indices, int32_t* counts,
                 void* workspace, size_t workspace_bytes, void* stream, const char* name);

}  // namespace
}  // namespace swattn

using namespace swattn;

extern "C" {

int swattn_version(void) { return (0 << 16) | 2; }

const char* swattn_last_error(void) { return g_last_error.c_str(); }

size_t swattn_compact_workspace_bytes(int64_t n) {
  const int64_t nb = ceil_div(n, kCompactChunk);
  return nb > 1 ? static_cast<size_t>(nb) * sizeof(int32_t) : 0;
}

int swattn_compact(const uint8_t* mask, int64_t n, int32_t* indices, int32_t* counts,
                   void* workspace, size_t workspace_bytes, void* stream) {
  return compact_impl(MaskSource{mask}, mask == nullptr, n, indices, counts, workspace,
                      workspace_bytes, stream, "swattn_compact");
}

int swattn_compact_logits(const void* logits, int32_t dtype, int64_t n, float threshold,
                          int32_t* indices, int32_t* counts, void* workspace,
                          size_t workspace_bytes, void* stream) {
  const char* name = "swattn_compact_logits";
  switch (dtype) {
    case SWATTN_DTYPE_F32:
      return compact_impl(F32LogitSource{static_cast<const float*>(logits), threshold},
                          logits == nullptr, n, indices, counts, workspace, workspace_bytes,
                          stream, name);
    case SWATTN_DTYPE_BF16:
      return compact_impl(BF16LogitSource{static_cast<const uint16_t*>(logits), threshold},
                          logits == nullptr, n, indices, counts, workspace, workspace_bytes,
                          stream, name);
    case SWATTN_DTYPE_F16:
      return compact_impl(F16LogitSource{static_cast<const _Float16*>(logits), threshold},
                          logits == nullptr, n, indices, counts, workspace, workspace_bytes,
                          stream, name);
    default:
      return invalid("swattn_compact_logits: dtype must be SWATTN_DTYPE_F32, _BF16 or _F16");
  }
}

int swattn_check_indices(const int32_t* full, int64_t n_full, const int32_t* local,
                         int64_t n_local, int64_t seq_len, int32_t* flags, void* stream) {
  if (n_full < 0 || n_local < 0 || seq_len < 0 || seq_len > INT32_MAX)
    return invalid("swattn_check_indices: bad sizes");
  if (flags == nullptr || (n_full > 0 && full == nullptr) || (n_local > 0 && local == nullptr))
    return invalid("swattn_check_indices: null pointer");
  const hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(flags_clear_kernel, dim3(1), dim3(1), 0, st, flags);
  const int64_t n = n_full > n_local ? n_full : n_local;
  if (n > 0) {
    hipLaunchKernelGGL(check_indices_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, st, full,
                       n_full, local, n_local, seq_len, flags);
  }
  return launch_status("swattn_check_indices");
}

int swattn_build_metadata(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv,
                          int32_t num_seqs, int64_t total_q, int64_t total_kv, int32_t window,
                          int32_t* q_positions, int32_t* kv_positions, int32_t* q_segment_ids,
                          int32_t* kv_segment_ids, int32_t* full_starts, int32_t* local_starts,
                          int32_t* causal_ends, void* stream) {
  if (num_seqs < 1 || total_q < 0 || total_kv < 0 || total_q > INT32_MAX || total_kv > INT32_MAX)
    return invalid("swattn_build_metadata: bad sizes");
  if (window <= 0) return invalid("swattn_build_metadata: window must be positive");
  if (cu_seqlens_q == nullptr || cu_seqlens_kv == nullptr)
    return invalid("swattn_build_metadata: null cu_seqlens");
  if ((total_q > 0 && (q_positions == nullptr || q_segment_ids == nullptr ||
                       full_starts == nullptr || local_starts == nullptr ||
                       causal_ends == nullptr)) ||
      (total_kv > 0 && (kv_positions == nullptr || kv_segment_ids == nullptr)))
    return invalid("swattn_build_metadata: null output");
  const int64_t n = total_q > total_kv ? total_q : total_kv;
  if (n == 0) return SWATTN_OK;
  hipLaunchKernelGGL(metadata_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, as_stream(stream),
                     cu_seqlens_q, cu_seqlens_kv, num_seqs, total_q, total_kv, window,
                     q_positions, kv_positions, q_segment_ids, kv_segment_ids, full_starts,
                     local_starts, causal_ends);
  return launch_status("swattn_build_metadata");
}

}  // extern "C"

namespace swattn {
namespace {

template <typename Src>
int compact_impl(const Src& src, bool src_null, int64_t n, int32_t* indices, int32_t* counts,
                 void* workspace, size_t workspace_bytes, void* stream, const char* name) {
  if (n < 0 || n > INT32_MAX) return invalid(std::string(name) + ": n must be in [0, 2^31)");
  if (counts == nullptr || (n > 0 && (src_null || indices == nullptr)))
    return invalid(std::string(name) + ": null pointer");
  const hipStream_t st = as_stream(stream);
  if (n == 0) {
    hipLaunchKernelGGL(flags_clear_kernel, dim3(1), dim3(1), 0, st, counts);
    hipLaunchKernelGGL(flags_clear_kernel, dim3(1), dim3(1), 0, st, counts + 1);
    return launch_status(name);
  }
  const int64_t nb = ceil_div(n, kCompactChunk);
  if (nb > 1) {
    if (workspace == nullptr || workspace_bytes < swattn_compact_workspace_bytes(n)) {
      set_error(std::string(name) + ": workspace too small");
      return SWATTN_EWORKSPACE;
    }
    if (!aligned256(workspace)) return invalid(std::string(name) + ": workspace must be 256-byte aligned");
    int32_t* bc = static_cast<int32_t*>(workspace);
    hipLaunchKernelGGL(compact_count_kernel<Src>, dim3(nb), dim3(kCompactThreads), 0, st, src, n,
                       bc);
    hipLaunchKernelGGL(compact_scatter_kernel<Src>, dim3(nb), dim3(kCompactThreads), 0, st, src,
                       n, static_cast<const int32_t*>(bc), static_cast<int>(nb), indices, counts);
  } else {
    hipLaunchKernelGGL(compact_scatter_kernel<Src>, dim3(1), dim3(kCompactThreads), 0, st, src, n,
                       static_cast<const int32_t*>(nullptr), 1, indices, counts);
  }
  return launch_status(name);
}

}  // namespace
}  // namespace swattn
