// Routed GQA decode for gfx950: one new query token per sequence attends its
// KV cache, either fully (causal over the whole cache) or over the last
// `window` keys -- the routing rule of the prefill path applied to its last
// row (F:145-155: query position p = len - 1 sees keys [0, p] when full and
// [p - window + 1, p] when local).  The reference has no decode path.
//
// HBM-bound: every cached key and value of the routed range is read once per
// KV head.  Split-K (workgroups each streaming one chunk of one sequence's
// routed keys with an online softmax) keeps the chip busy for one long
// sequence as well as for many short ones.  Which keys are routed is known
// only on the device, so a one-workgroup plan kernel sums the routed key
// counts, picks one chunk size for the whole launch, and writes the list of
// (sequence, KV head, chunk) work items: full and local sequences then get
// chunks of the same size, whatever the mix.  A third kernel merges the
// fp32 split partials in the log2 domain (LSE as V:236-241).
//
// Layout: q [B, Hq, 128], caches [B, L, Hkv, 128] bf16; out [B, Hq, 128] bf16,
// lse [B, Hq] fp32.  Group size G = Hq / Hkv <= 8.

#include <math.h>

#include <mutex>
#include <string>

#include "common.h"

namespace swattn {
namespace {

constexpr int kD = 128;
constexpr int kDecWaves = 4;         // waves per workgroup
constexpr int kMaxG = 8;
constexpr int kMaxSplitsDev = 256;   // splits per (sequence, KV head), at most

struct DecodeParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* lens;
  const uint8_t* full;
  float* part_o;     // [split][G][128] unnormalised sum of p * v, per work item
  float* part_ml;    // [split][G][2]   split max (exp2 domain) and sum of p
  int2* items;       // [split] (pair = b * Hkv + kvh, chunk index)   (plan output)
  int64_t* plan;     // [0] chunk keys, [1] work items; [2 + 2b] first item of b, [3 + 2b] chunks of b
  uint16_t* out;
  float* lse;
  int64_t cache_len; // L
  int batch, hq, hkv, group, window;
  int max_items;     // grid size of the split kernel (an upper bound on the work items)
  int target;        // work items the chunk size aims at
  float c;           // sm_scale * log2(e)
};

__device__ __forceinline__ float bf(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Sum over each row of 16 lanes, every lane getting the row's sum, with DPP
// moves only (no LDS round trip): swap neighbours, swap pairs, then add the
// mirror image within 8 and within 16 lanes.
__device__ __forceinline__ float row16_sum(float x) {
  constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kHalfMirror = 0x141, kMirror = 0x140;
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kXor1, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kXor2, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kHalfMirror, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kMirror, 0xf, 0xf, false));
  return x;
}

// Key range of sequence b: [lo, hi).
__device__ __forceinline__ void key_range(const DecodeParams& p, int b, int64_t& lo, int64_t& hi) {
  int64_t len = p.lens[b];
  len = len < 0 ? 0 : (len > p.cache_len ? p.cache_len : len);
  hi = len;
  lo = p.full[b] ? 0 : (len - p.window > 0 ? len - p.window : 0);
}

// Plan: one workgroup of 1024 threads.  T = total routed keys over all
// (sequence, KV head) pairs; chunk = max(256, ceil(T / target),
// ceil(L / 256)) rounded up to 16, so that there are at most target + pairs
// work items and at most 256 per pair; sequence b gets ceil(keys_b / chunk)
// chunks per KV head.  Work items are numbered sequence by sequence, KV head
// by KV head, chunk by chunk.
constexpr int kPlanThreads = 1024;
constexpr int kPlanLdsSeqs = 4096;   // sequences whose first item and chunk count stay in LDS
__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(const DecodeParams p) {
  __shared__ int64_t s_red[kPlanThreads / 64];
  __shared__ int64_t s_scan[kPlanThreads];
  __shared__ int32_t s_first[kPlanLdsSeqs], s_n[kPlanLdsSeqs];
  const bool in_lds = p.batch <= kPlanLdsSeqs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (p.batch + kPlanThreads - 1) / kPlanThreads;
  const int b0 = min(tid * per, p.batch), b1 = min(b0 + per, p.batch);
  int64_t keys = 0;
  for (int b = b0; b < b1; ++b) {
    int64_t lo, hi;
    key_range(p, b, lo, hi);
    keys += hi - lo;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) keys += __shfl_xor(keys, off);
  if (lane == 0) s_red[wave] = keys;
  __syncthreads();
  int64_t total = 0;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) total += s_red[w];
  total *= p.hkv;
  int64_t chunk = (total + p.target - 1) / p.target;
  const int64_t by_len = (p.cache_len + 255) / 256;
  chunk = chunk > by_len ? chunk : by_len;
  chunk = chunk > 256 ? chunk : 256;
  chunk = (chunk + 15) & ~static_cast<int64_t>(15);
  int64_t cnt = 0;
  for (int b = b0; b < b1; ++b) {
    int64_t lo, hi;
    key_range(p, b, lo, hi);
    cnt += (hi - lo + chunk - 1) / chunk;
  }
  // Inclusive scan of the per-thread chunk counts (Hillis-Steele in LDS).
  s_scan[tid] = cnt;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int64_t add = tid >= off ? s_scan[tid - off] : 0;
    __syncthreads();
    s_scan[tid] += add;
    __syncthreads();
  }
  int64_t run = s_scan[tid] - cnt;   // chunks (per KV head) before sequence b0
  for (int b = b0; b < b1; ++b) {
    int64_t lo, hi;
    key_range(p, b, lo, hi);
    const int64_t n = (hi - lo + chunk - 1) / chunk;
    p.plan[2 + 2 * b] = run * p.hkv;
    p.plan[3 + 2 * b] = n;
    if (in_lds) {
      s_first[b] = static_cast<int32_t>(run * p.hkv);
      s_n[b] = static_cast<int32_t>(n);
    }
    run += n;
  }
  const int64_t items = s_scan[kPlanThreads - 1] * p.hkv;
  if (tid == 0) {
    p.plan[0] = chunk;
    p.plan[1] = items;
  }
  __syncthreads();   // every sequence's first item and chunk count are written
  // Work items, one per thread at a time: item i belongs to the last
  // sequence whose first item is <= i (sequences without keys own none).
  // The search runs in LDS when the sequences fit there (item counts stay
  // below 2^31: at most target + pairs).
  for (int64_t i = tid; i < items; i += kPlanThreads) {
    int lo = 0, hi = p.batch - 1;
    if (in_lds) {
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_first[mid] <= i) lo = mid; else hi = mid - 1;
      }
    } else {
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (p.plan[2 + 2 * mid] <= i) lo = mid; else hi = mid - 1;
      }
    }
    const int64_t r = i - (in_lds ? s_first[lo] : p.plan[2 + 2 * lo]);
    const int64_t n = in_lds ? s_n[lo] : p.plan[3 + 2 * lo];
    const int kvh = static_cast<int>(r / n);
    p.items[i] = make_int2(lo * p.hkv + kvh, static_cast<int>(r - static_cast<int64_t>(kvh) * n));
  }
}

// One workgroup per work item (a chunk of `chunk` keys of one sequence's
// routed range, for one KV head).  Lane l works on the keys of key group kg = l / 16 and on
// dims 8*(l%16) .. +7: wave w takes the keys 16*i + 4*w + kg of its split, so
// the four waves sweep the split together, four keys per wave per step.
// Each key group keeps its own online-softmax state (running max m, sum l,
// unnormalised sum acc of p * v) for every head of the group; the max moves
// only when a score exceeds it by more than 8 in the exp2 domain, so the
// state is rarely rescaled (the prefill kernel's rule).  The groups and
// waves are combined at the end into one partial per workgroup.
template <int G>
__global__ __launch_bounds__(256) void decode_split_kernel(const DecodeParams p) {
  __shared__ float s_m[kDecWaves][G], s_l[kDecWaves][G];
  __shared__ float s_acc[kDecWaves][G][kD];
  const int64_t slot = blockIdx.x;
  if (slot >= p.plan[1]) return;   // beyond the planned work items
  const int2 item = p.items[slot];
  const int b = item.x / p.hkv, kvh = item.x - (item.x / p.hkv) * p.hkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kg = lane >> 4, ds = lane & 15;
  int64_t lo, hi;
  key_range(p, b, lo, hi);
  const int64_t chunk = p.plan[0];
  const int64_t k0 = lo + static_cast<int64_t>(item.y) * chunk;
  const int64_t k1 = k0 + chunk < hi ? k0 + chunk : hi;
  float* po = p.part_o + slot * G * kD;
  float* pml = p.part_ml + slot * G * 2;
  if (k0 >= k1) {   // no key of this sequence in the split: an empty partial
    if (tid < G) {
      pml[2 * tid] = -INFINITY;
      pml[2 * tid + 1] = 0.f;
    }
    return;
  }
  // Q rows of the group: dims 8*ds .. +7 of each head, in fp32, pre-scaled
  // by c so that a dot product is already the exp2-domain score.
  float qv[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint4 u = *reinterpret_cast<const uint4*>(
        p.q + (static_cast<int64_t>(b) * p.hq + kvh * G + h) * kD + 8 * ds);
    const uint32_t x[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qv[h][2 * e] = bf(x[e] & 0xffffu) * p.c;
      qv[h][2 * e + 1] = bf(x[e] >> 16) * p.c;
    }
  }
  const int64_t row_stride = static_cast<int64_t>(p.hkv) * kD;   // elements per cache row
  const uint16_t* kb = p.k + (static_cast<int64_t>(b) * p.cache_len) * row_stride + kvh * kD + 8 * ds;
  const uint16_t* vb = p.v + (static_cast<int64_t>(b) * p.cache_len) * row_stride + kvh * kD + 8 * ds;

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }
  // Keys of this lane: first = k0 aligned down to 16, then every 16.
  const int64_t base = (k0 & ~static_cast<int64_t>(15)) + 4 * wave + kg;
  const int64_t steps = (k1 - (k0 & ~static_cast<int64_t>(15)) + 15) >> 4;
  // Loads run kPf steps ahead of the compute (a ring of registers, the loop
  // unrolled by kPf so that every slot is static): one step alone is four
  // keys per wave, far too little to cover HBM latency.
  constexpr int kPf = G <= 4 ? 8 : 4;
  auto load = [&](int64_t i, uint4& kv, uint4& vv) {
    int64_t key = base + 16 * i;
    key = key < k0 ? k0 : (key >= k1 ? k1 - 1 : key);   // in bounds; masked below
    kv = *reinterpret_cast<const uint4*>(kb + key * row_stride);
    vv = *reinterpret_cast<const uint4*>(vb + key * row_stride);
  };
  uint4 kr[kPf], vr[kPf];
#pragma unroll
  for (int j = 0; j < kPf; ++j) load(j, kr[j], vr[j]);
  for (int64_t i0 = 0; i0 < steps; i0 += kPf) {
#pragma unroll
    for (int j = 0; j < kPf; ++j) {
      const int64_t i = i0 + j;
      if (i >= steps) break;
      const int64_t key = base + 16 * i;
      const bool live = key >= k0 && key < k1;
      const uint32_t kx[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
      float s[G];
#pragma unroll
      for (int h = 0; h < G; ++h) s[h] = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a0 = bf(kx[e] & 0xffffu), a1 = bf(kx[e] >> 16);
#pragma unroll
        for (int h = 0; h < G; ++h)
          s[h] = __builtin_fmaf(a1, qv[h][2 * e + 1], __builtin_fmaf(a0, qv[h][2 * e], s[h]));
      }
      bool moved = false;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        s[h] = row16_sum(s[h]);
        if (!live) s[h] = -INFINITY;
        moved = moved || (s[h] - m[h] > 8.0f);
      }
      if (__builtin_amdgcn_ballot_w64(moved)) {   // rare: move the maxima, rescale
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float mn = s[h] - m[h] > 8.0f ? s[h] : m[h];
          const float a = mn == m[h] ? 1.0f : __builtin_amdgcn_exp2f(m[h] - mn);
          m[h] = mn;
          l[h] *= a;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] *= a;
        }
      }
      const uint32_t vx[4] = {vr[j].x, vr[j].y, vr[j].z, vr[j].w};
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pr = live ? __builtin_amdgcn_exp2f(s[h] - m[h]) : 0.f;
        l[h] += pr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[h][2 * e] = __builtin_fmaf(pr, bf(vx[e] & 0xffffu), acc[h][2 * e]);
          acc[h][2 * e + 1] = __builtin_fmaf(pr, bf(vx[e] >> 16), acc[h][2 * e + 1]);
        }
      }
      load(i + kPf, kr[j], vr[j]);   // refill the slot; past the end: clamped, never used
    }
  }
  // Combine the four key groups of the wave (lanes l, l^16, l^32, l^48 hold
  // the same dims of different keys).
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mm = m[h];
    mm = fmaxf(mm, __shfl_xor(mm, 16));
    mm = fmaxf(mm, __shfl_xor(mm, 32));
    const float a = mm == -INFINITY ? 0.f : exp2f(m[h] - mm);
    float lh = l[h] * a;
    lh += __shfl_xor(lh, 16);
    lh += __shfl_xor(lh, 32);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = acc[h][e] * a;
      x += __shfl_xor(x, 16);
      x += __shfl_xor(x, 32);
      if (kg == 0) s_acc[wave][h][8 * ds + e] = x;
    }
    if (lane == 0) {
      s_m[wave][h] = mm;
      s_l[wave][h] = lh;
    }
  }
  __syncthreads();
  // Combine the waves: one partial (unnormalised acc, max, sum) per head.
  for (int i = tid; i < G * kD; i += 256) {
    const int h = i / kD, d = i - h * kD;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) mm = fmaxf(mm, s_m[w][h]);
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w)
      if (s_m[w][h] != -INFINITY) a += exp2f(s_m[w][h] - mm) * s_acc[w][h][d];
    po[i] = a;
  }
  if (tid < G) {
    float mm = -INFINITY, lh = 0.f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) mm = fmaxf(mm, s_m[w][tid]);
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w)
      if (s_m[w][tid] != -INFINITY) lh += exp2f(s_m[w][tid] - mm) * s_l[w][tid];
    pml[2 * tid] = mm;
    pml[2 * tid + 1] = lh;
  }
}

// One workgroup per output row (b, head): merge the split partials.  Every
// thread takes a share of the splits for the maximum and the weighted sum,
// then thread t accumulates dim t % 128 over its half of the splits, eight
// independent loads in flight.
__global__ __launch_bounds__(256) void decode_merge_kernel(const DecodeParams p) {
  __shared__ float s_w[kMaxSplitsDev];
  __shared__ float s_red[8];
  __shared__ float s_half[kD];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = static_cast<int>(row / p.hq), hq = static_cast<int>(row - static_cast<int64_t>(b) * p.hq);
  const int kvh = hq / p.group, h = hq - kvh * p.group;
  const int nch = static_cast<int>(p.plan[3 + 2 * b]);   // at most 256
  const int64_t slot0 = p.plan[2 + 2 * b] + static_cast<int64_t>(kvh) * nch;
  // Maximum over the non-empty splits.
  float mx = -INFINITY;
  for (int c = tid; c < nch; c += 256) {
    const float* ml = p.part_ml + ((slot0 + c) * p.group + h) * 2;
    if (ml[1] > 0.f) mx = fmaxf(mx, ml[0]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  // Split weights 2^(m_c - M) (0 for empty splits) and the weighted sum of l.
  float lsum = 0.f;
  for (int c = tid; c < nch; c += 256) {
    const float* ml = p.part_ml + ((slot0 + c) * p.group + h) * 2;
    const float w = (ml[1] > 0.f && M != -INFINITY) ? __builtin_amdgcn_exp2f(ml[0] - M) : 0.f;
    s_w[c] = w;
    lsum += w * ml[1];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) lsum += __shfl_xor(lsum, off);
  if (lane == 0) s_red[4 + wave] = lsum;
  __syncthreads();
  const float L = s_red[4] + s_red[5] + s_red[6] + s_red[7];
  // Weighted sum of the unnormalised partial outputs.
  const int d = tid & (kD - 1), half = tid >> 7;
  const float* base = p.part_o + (slot0 * p.group + h) * kD + d;
  const int64_t cstride = static_cast<int64_t>(p.group) * kD;
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int c = half;
  for (; c + 14 < nch; c += 16) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float w = s_w[c + 2 * u];
      if (w != 0.f) a[u] += w * base[(c + 2 * u) * cstride];
    }
  }
  for (; c < nch; c += 2) {
    const float w = s_w[c];
    if (w != 0.f) a[0] += w * base[c * cstride];
  }
  float acc = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  if (half == 1) s_half[d] = acc;
  __syncthreads();
  if (half == 0) {
    acc += s_half[d];
    const float o = acc / L;   // empty row: 0 / 0 = NaN, as the prefill writes it
    p.out[row * kD + d] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(o));
    if (d == 0) p.lse[row] = M == -INFINITY ? -INFINITY : M + log2f(L);
  }
}

}  // namespace
}  // namespace swattn

using namespace swattn;

extern "C" {

// Work items the chunk size aims at: about four workgroups per CU.  The
// split kernel's grid is that plus one per (sequence, KV head) pair, an
// upper bound on the planned items (rounding each pair's chunk count up).
#ifndef SWATTN_SPLIT_TARGET
#define SWATTN_SPLIT_TARGET 4
#endif
constexpr int kSplitTarget = SWATTN_SPLIT_TARGET;   // workgroups per CU

static int decode_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}

struct DecodeLayout {
  int64_t target, max_items, off_ml, off_items, off_plan, bytes;   // byte offsets
};

static DecodeLayout decode_layout(int64_t batch, int64_t heads_q, int64_t heads_kv, int cus) {
  DecodeLayout L{};
  L.target = static_cast<int64_t>(kSplitTarget) * cus;
  L.max_items = L.target + batch * heads_kv;
  const int64_t group = heads_q / heads_kv;
  auto al = [](int64_t x) { return (x + 255) & ~static_cast<int64_t>(255); };
  int64_t o = al(L.max_items * group * kD * 4);           // part_o
  L.off_ml = o;    o = al(o + L.max_items * group * 2 * 4);
  L.off_items = o; o = al(o + L.max_items * 8);
  L.off_plan = o;  o = al(o + (2 + 2 * batch) * 8);
  L.bytes = o;
  return L;
}

size_t swattn_decode_workspace_bytes(int32_t batch, int64_t cache_len, int32_t heads_q,
                                     int32_t heads_kv) {
  if (batch < 1 || cache_len < 1 || heads_q < 1 || heads_kv < 1 || heads_q % heads_kv) return 0;
  return static_cast<size_t>(decode_layout(batch, heads_q, heads_kv, decode_cus()).bytes);
}

}  // extern "C"

// Argument checks shared by both decode entry points (name = the entry point).
static int decode_check(const char* name, const void* q, const void* k_cache,
                        const void* v_cache, const int32_t* cache_lens, const uint8_t* full,
                        void* out, float* lse, int32_t batch, int64_t cache_len,
                        int32_t heads_q, int32_t heads_kv, int32_t head_dim, int32_t window) {
  const std::string n(name);
  if (head_dim != kD) return invalid(n + ": head_dim must be 128");
  if (batch < 1 || cache_len < 1 || heads_q < 1 || heads_kv < 1) return invalid(n + ": bad shape");
  if (heads_q % heads_kv) return invalid(n + ": heads_q must be a multiple of heads_kv");
  if (heads_q / heads_kv > kMaxG) return invalid(n + ": heads_q / heads_kv must be at most 8");
  if (window <= 0) return invalid(n + ": window must be positive");
  if (batch > 65535 || heads_kv > 65535 || cache_len > INT32_MAX ||
      static_cast<int64_t>(batch) * heads_q > INT32_MAX)
    return invalid(n + ": batch, heads_kv or cache_len too large");
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr || cache_lens == nullptr ||
      full == nullptr || out == nullptr || lse == nullptr)
    return invalid(n + ": null pointer");
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
    return invalid(n + ": q, k_cache, v_cache and out must be 16-byte aligned");
  return SWATTN_OK;
}

// Plan, split and merge kernels on `stream` with the (checked) workspace ws.
static int decode_launch(const char* name, const void* q, const void* k_cache,
                         const void* v_cache, const int32_t* cache_lens, const uint8_t* full,
                         void* out, float* lse, int32_t batch, int64_t cache_len,
                         int32_t heads_q, int32_t heads_kv, int32_t window, float scale_log2,
                         char* ws, void* stream) {
  const int group = heads_q / heads_kv;
  DecodeParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k_cache);
  p.v = static_cast<const uint16_t*>(v_cache);
  p.lens = cache_lens;
  p.full = full;
  const DecodeLayout L = decode_layout(batch, heads_q, heads_kv, decode_cus());
  if (L.max_items > INT32_MAX) return invalid(std::string(name) + ": too many work items");
  p.part_o = reinterpret_cast<float*>(ws);
  p.part_ml = reinterpret_cast<float*>(ws + L.off_ml);
  p.items = reinterpret_cast<int2*>(ws + L.off_items);
  p.plan = reinterpret_cast<int64_t*>(ws + L.off_plan);
  p.max_items = static_cast<int>(L.max_items);
  p.target = static_cast<int>(L.target);
  p.batch = batch;
  p.out = static_cast<uint16_t*>(out);
  p.lse = lse;
  p.cache_len = cache_len;
  p.hq = heads_q;
  p.hkv = heads_kv;
  p.group = group;
  p.window = window;
  p.c = scale_log2;
  const hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, st, p);
  const dim3 grid(static_cast<uint32_t>(p.max_items));
  switch (group) {
    case 1: hipLaunchKernelGGL(decode_split_kernel<1>, grid, dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL(decode_split_kernel<2>, grid, dim3(256), 0, st, p); break;
    case 3: hipLaunchKernelGGL(decode_split_kernel<3>, grid, dim3(256), 0, st, p); break;
    case 4: hipLaunchKernelGGL(decode_split_kernel<4>, grid, dim3(256), 0, st, p); break;
    case 5: hipLaunchKernelGGL(decode_split_kernel<5>, grid, dim3(256), 0, st, p); break;
    case 6: hipLaunchKernelGGL(decode_split_kernel<6>, grid, dim3(256), 0, st, p); break;
    case 7: hipLaunchKernelGGL(decode_split_kernel<7>, grid, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL(decode_split_kernel<8>, grid, dim3(256), 0, st, p); break;
  }
  const int64_t rows = static_cast<int64_t>(batch) * heads_q;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, st, p);
  return launch_status(name);
}

extern "C" {

int swattn_decode_fwd(const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* cache_lens, const uint8_t* full, void* out, float* lse,
                      int32_t batch, int64_t cache_len, int32_t heads_q, int32_t heads_kv,
                      int32_t head_dim, int32_t window, float scale_log2, void* workspace,
                      size_t workspace_bytes, void* stream) {
  const char* name = "swattn_decode_fwd";
  const int st = decode_check(name, q, k_cache, v_cache, cache_lens, full, out, lse, batch,
                              cache_len, heads_q, heads_kv, head_dim, window);
  if (st != SWATTN_OK) return st;
  const size_t need = swattn_decode_workspace_bytes(batch, cache_len, heads_q, heads_kv);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("swattn_decode_fwd: workspace smaller than swattn_decode_workspace_bytes()");
    return SWATTN_EWORKSPACE;
  }
  if (!aligned256(workspace)) return invalid("swattn_decode_fwd: workspace must be 256-byte aligned");
  return decode_launch(name, q, k_cache, v_cache, cache_lens, full, out, lse, batch, cache_len,
                       heads_q, heads_kv, window, scale_log2, static_cast<char*>(workspace),
                       stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The same decode with library-owned scratch, for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops).
// `scratch` is a file-scope device array: every GPU the library runs on gets
// its own copy, held until the process ends.  In host code its name is only a
// host-side stand-in, so its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// ever handed to kernels.  The decode kernels write every scratch byte they
// read within the same call (plan, work items, split partials), so nothing
// needs clearing between calls; two calls that overlap on one GPU share the
// array and race.
// ---------------------------------------------------------------------------
constexpr size_t kDecodeScratchBytes = SWATTN_DECODE_NOALLOC_MAX_BYTES;   // 16 MiB per GPU
static_assert(kDecodeScratchBytes % 256 == 0, "whole 256-byte lines");
static __device__ __align__(256) char scratch[kDecodeScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];   // per device, nullptr until looked up

// Device address of this GPU's scratch array (the current device's), or
// nullptr with the error set.
static void* scratch_for_current_device(const char* name) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    set_error(std::string(name) + ": no usable current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error(std::string(name) + ": hipGetSymbolAddress(scratch): " + hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

extern "C" {

int swattn_decode_fwd_noalloc(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* cache_lens, const uint8_t* full, void* out,
                              float* lse, int32_t batch, int64_t cache_len, int32_t heads_q,
                              int32_t heads_kv, int32_t head_dim, int32_t window,
                              float scale_log2, void* stream) {
  const char* name = "swattn_decode_fwd_noalloc";
  const int st = decode_check(name, q, k_cache, v_cache, cache_lens, full, out, lse, batch,
                              cache_len, heads_q, heads_kv, head_dim, window);
  if (st != SWATTN_OK) return st;
  const size_t need = swattn_decode_workspace_bytes(batch, cache_len, heads_q, heads_kv);
  if (need > kDecodeScratchBytes) {
    set_error("swattn_decode_fwd_noalloc: this shape needs " + std::to_string(need) +
              " bytes of scratch, more than the library's " +
              std::to_string(kDecodeScratchBytes) + " (use swattn_decode_fwd with a workspace)");
    return SWATTN_EINVAL;
  }
  void* ws = scratch_for_current_device(name);
  if (ws == nullptr) return SWATTN_EINVAL;
  return decode_launch(name, q, k_cache, v_cache, cache_lens, full, out, lse, batch, cache_len,
                       heads_q, heads_kv, window, scale_log2, static_cast<char*>(ws), stream);
}

}  // extern "C"
