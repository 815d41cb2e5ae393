// Routed GQA prefill forward for gfx950 (MI355X): both Switch Attention
// branches in a single launch.
//
// Reference tags: V = swiattn_gqa_prefill_varlen.py, F = swiattn_gqa_prefill.py.
// Semantics follow the reference branch kernel (V:103-249): per query row a
// half-open key range [start, end) (V:134-137, V:186-196; F:145-155 without
// metadata), raw scores s = q.k, online softmax in base 2 with
// c = sm_scale*log2(e) (V:73-76, V:207-221), P rounded to bf16 before P.V
// while the row sum uses the fp32 P (V:219-225), a finite -2^30 max sentinel
// (V:174), O = acc / l and LSE = log2(l) + m*c (V:236-241), and O/LSE written
// only to the routed rows (V:243-249).
//
// Design (MI355X-first, not a translation of the TileLang schedule):
// * Work item = (branch, tile of 256 "rows", KV head).  A row is a
//   (compacted query slot, query head of the KV head's group) pair with the
//   head index fastest, so one K/V tile in LDS serves every query head of the
//   group (GQA packing) and a wave's rows span only 64/G query positions.
// * The whole routed problem is one grid: full-branch tiles first, last tile
//   (longest causal prefix) first, then local tiles; KV head = item % Hkv so
//   that with Hkv = 8 every XCD (blockIdx % 8) streams a single KV head
//   through its own L2.  Counts come from the index lists' lengths, so new
//   routing never recompiles anything.
// * Eight waves share each K/V tile; each wave owns 32 rows and computes
//   S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (Q^T stays in registers as the
//   B operand).  Two waves per SIMD let one wave's softmax (VALU) run under
//   the other's MFMAs, and every accumulator stays in ordinary VGPRs.  Each
//   lane owns one query row and 32 keys of the 64-key tile: row max and row
//   sum are lane-local plus one permlane32 swap.  The S^T accumulator is
//   already the B operand of O^T = V^T P^T (keys permuted consistently on
//   both sides), and V^T operands come straight from the row-major V tile
//   with ds_read_b64_tr_b16.
// * K/V tiles stream global -> LDS with global_load_lds_dwordx4 (no register
//   staging) through three LDS stages, two tiles ahead of the compute, with
//   one barrier per tile.  The loads are issued from inline assembly and
//   waited for with explicit vmcnt counts: the compiler cannot see that they
//   target another stage than the one being read, and would otherwise drain
//   every load before each LDS read.  LDS rows are unpadded 256-byte rows
//   whose 16-byte chunks are XOR-swizzled so both operand read patterns are
//   conflict-free.
// * The running max is only moved when it grows by more than 2^8 in the
//   exp2 domain (rescaling O is then rare); P = 2^(s*c - m*c) stays below
//   2^8, and O = acc / l, LSE = log2(l) + m*c are the same quantities as with
//   an exact running max.
// * Tiles outside a wave's key range are skipped and interior tiles skip the
//   mask.

#include <limits.h>
#include <math.h>

#include "common.h"

namespace swattn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kD = 128;                               // head_dim
constexpr int kBN = 64;                               // keys per K/V tile
constexpr int kWaves = 8;                             // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kRowsPerWave = 32;                      // one 32-row MFMA block
constexpr int kRowsPerItem = kWaves * kRowsPerWave;   // 256 rows per work item
constexpr int kRowBytes = kD * 2;                     // 256-byte key rows, unpadded
constexpr int kTileBytes = kBN * kRowBytes;           // one K or V tile: 16 KiB
constexpr int kStageBytes = 2 * kTileBytes;           // K + V
constexpr int kStages = 3;
constexpr int kLdsBytes = kStages * kStageBytes;      // 96 KiB
constexpr int kLoadsPerTile = 4;                      // global_load_lds per thread per tile
static_assert(kLoadsPerTile == 4, "the vmcnt(4) waits in fwd_kernel assume 4 loads per tile");
constexpr float kMaxSentinel = -1073741824.0f;        // -2^30 (V:174)

struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  float* lse;
  const int32_t* idx[2];     // [0] full list, [1] local list
  const int32_t* starts[2];  // metadata starts per branch (kMeta only)
  const int32_t* ends;       // metadata causal ends (kMeta only)
  int32_t count[2];
  int32_t tiles[2];
  int32_t seq_q, seq_kv, total_kv;
  int32_t hq, hkv, group, window;
  float c;                   // sm_scale * log2(e)
};

// Chunk swizzle: logical 16-byte chunk j of key row r lives at chunk
// j ^ swz(r).  swz is a permutation of r mod 16, so 16 lanes reading one
// chunk of 16 consecutive rows hit 16 distinct bank groups, and the four
// rows x four chunks touched by 32 lanes of a transposing V read are 16
// distinct chunks as well.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ float xor32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ int wave_min(int x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = min(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = max(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const __bf16 ha = static_cast<__bf16>(a), hb = static_cast<__bf16>(b);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, ha)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
}
__device__ __forceinline__ i16x4 lds_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)((__attribute__((address_space(3))) char*)(p)));
}
// 16 bytes per lane from global memory to LDS at lds_base + 16 * lane
// (global_load_lds_dwordx4; the LDS base goes through M0 and must be
// wave-uniform).  Issued as inline assembly so that the compiler's wait
// insertion does not treat it as a store that aliases every LDS read.
__device__ __forceinline__ void dma16(const uint16_t* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// Stage one 64-key K and V tile: wave w fills key rows 8w .. 8w+7.  Load i
// of a wave writes rows 8w+4i .. +3 (1 KiB, lane-linear); lane l lands on
// chunk position l%16 of row l/16 and therefore fetches logical chunk
// (l%16) ^ swz(row) from global memory.  Issues kLoadsPerTile loads per lane.
__device__ __forceinline__ void stage_tile(const FwdParams& p, const char* stage, int key0,
                                           int kvh, int wave, int lane) {
  const int sub = lane >> 4, pcol = lane & 15;
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(stage) + 8 * wave * kRowBytes);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 8 * wave + 4 * i + sub;
    const int j = pcol ^ swz(row);
    const int key = min(key0 + row, p.total_kv - 1);
    const int64_t off = (static_cast<int64_t>(key) * p.hkv + kvh) * kD + 8 * j;
    dma16(p.k + off, base + 4 * i * kRowBytes);
    dma16(p.v + off, base + 4 * i * kRowBytes + kTileBytes);
  }
}

template <bool kMeta>
__device__ __forceinline__ void row_bounds(const FwdParams& p, int branch, int pos, int& ks,
                                           int& ke) {
  if constexpr (kMeta) {
    ks = p.starts[branch][pos];
    ke = p.ends[pos];
  } else {
    const int b = pos / p.seq_q;
    const int i = pos - b * p.seq_q;
    const int base = b * p.seq_kv;
    ke = base + min(i + 1, p.seq_kv);
    ks = branch == 0 ? base : base + max(i - p.window + 1, 0);
  }
  ks = max(ks, 0);
  ke = min(ke, p.total_kv);
}

// Keys held by this lane in a 32-key S^T block: 8*j + 4*hh + i (register 4j+i).
__device__ __forceinline__ void mask_block(f32x16& s, int key0, int hh, int ks, int ke) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = key0 + 8 * j + 4 * hh + i;
      if (key < ks || key >= ke) s[4 * j + i] = -INFINITY;
    }
  }
}

// Online-softmax step of one 32-row x 64-key tile held as two S^T blocks.
// The max m only moves when the tile max exceeds it by more than 8 in the
// exp2 domain (or m is still the sentinel); alpha is then the O rescale
// factor, otherwise exactly 1.  Overwrites s0/s1 with P = 2^(s*c - m*c)
// (fp32) and returns whether m moved.
__device__ __forceinline__ bool softmax_step(f32x16& s0, f32x16& s1, float& m, float& l, float c,
                                             float& alpha) {
  float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
  for (int e = 1; e < 16; ++e) mx = fmaxf(mx, fmaxf(s0[e], s1[e]));
  mx = xor32_max(mx);
  const bool moved = (mx - m) * c > 8.0f;
  const float m_new = moved ? mx : m;
  alpha = moved ? __builtin_amdgcn_exp2f((m - m_new) * c) : 1.0f;
  const float mc = m_new * c;
  float rs0 = 0.f, rs1 = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    s0[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[e], c, -mc));
    s1[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[e], c, -mc));
    rs0 += s0[e];
    rs1 += s1[e];
  }
  const float rs = xor32_sum(rs0 + rs1);
  l = l * alpha + rs;
  m = m_new;
  return moved;
}

template <bool kMeta>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(2, 2))) void fwd_kernel(const FwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
  __shared__ int s_range[2 * kWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rl = lane & 31, hh = lane >> 5;

  // ---- work item -> (branch, tile, kv head) --------------------------------
  const int item = blockIdx.x;
  const int kvh = item % p.hkv;
  const int t = item / p.hkv;
  const int branch = t < p.tiles[0] ? 0 : 1;
  const int tile = branch == 0 ? p.tiles[0] - 1 - t : t - p.tiles[0];
  const int32_t* __restrict__ idx = p.idx[branch];
  const int count = p.count[branch];
  const int G = p.group;

  // ---- this lane's row ------------------------------------------------------
  const int r = tile * kRowsPerItem + wave * kRowsPerWave + rl;
  const int slot = r / G;
  const int qh = kvh * G + (r - slot * G);
  const bool valid = slot < count;
  const int pos = idx[valid ? slot : count - 1];
  int ks, ke;
  row_bounds<kMeta>(p, branch, pos, ks, ke);

  // ---- key ranges: wave union / intersection, workgroup union --------------
  const int w_min_s = wave_min(valid ? ks : INT_MAX);
  const int w_max_e = wave_max(valid ? ke : INT_MIN);
  const int w_max_s = wave_max(valid ? ks : INT_MIN);
  const int w_min_e = wave_min(valid ? ke : INT_MAX);
  if (lane == 0) {
    s_range[wave] = w_min_s;
    s_range[kWaves + wave] = w_max_e;
  }
  __syncthreads();
  int g_s = INT_MAX, g_e = INT_MIN;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    g_s = min(g_s, s_range[w]);
    g_e = max(g_e, s_range[kWaves + w]);
  }
  const int t_begin = g_s / kBN;
  const int t_end = g_e > g_s ? (g_e + kBN - 1) / kBN : t_begin;

  // ---- Q row as MFMA B operands (Q^T[d][row]); wait before any LDS load -----
  bf16x8 qf[8];
  {
    const uint16_t* qrow = p.q + (static_cast<int64_t>(pos) * p.hq + qh) * kD + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(qrow + 16 * kk);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- prologue: two tiles in flight -----------------------------------------
  if (t_begin < t_end) stage_tile(p, smem, t_begin * kBN, kvh, wave, lane);
  if (t_begin + 1 < t_end) stage_tile(p, smem + kStageBytes, (t_begin + 1) * kBN, kvh, wave, lane);

  f32x16 o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) o[d] = f32x16{};
  float m = kMaxSentinel, l = 0.f;
  const float c = p.c;
  bool o_zero = true;  // O is still exactly zero: a rescale can be skipped

  // Per-lane LDS byte offsets inside a stage.
  // K operand (A of S^T): key row 32*kb + rl, logical chunk 2*kk + hh.
  const int kx = hh ^ swz(rl);
  // V operand (A of O^T, transposing read): key rows 16*s2 + vrow (+8),
  // logical chunk 4*d + cq, 8-byte half (lane & 1).
  const int g16 = lane >> 4, i16 = lane & 15;
  const int cq = 2 * (g16 & 1) + ((i16 & 3) >> 1);
  const int vrow = 4 * hh + (i16 >> 2);
  const int vsw0 = swz(vrow), vsw1 = swz(vrow + 8);

  int stage = 0;
  for (int tk = t_begin; tk < t_end; ++tk) {
    // This lane's loads of tile tk are the oldest outstanding ones; after the
    // barrier every lane's are, and every wave has finished reading the stage
    // that the loads issued next will overwrite.
    if (tk + 1 < t_end)
      asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (tk + 2 < t_end) {
      const int s2i = stage == 0 ? 2 : stage - 1;
      stage_tile(p, smem + s2i * kStageBytes, (tk + 2) * kBN, kvh, wave, lane);
    }
    const int key0 = tk * kBN;
    if (key0 < w_max_e && key0 + kBN > w_min_s) {
      const char* kb = smem + stage * kStageBytes;
      const char* vb = kb + kTileBytes;
      // S^T = K Q^T: two 32-key blocks.
      f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int off = rl * kRowBytes + (((2 * kk) ^ kx) << 4);
        const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(kb + off);
        const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(kb + off + 32 * kRowBytes);
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[kk], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[kk], s1, 0, 0, 0);
      }
      if (!(key0 >= w_max_s && key0 + kBN <= w_min_e)) {
        mask_block(s0, key0, hh, ks, ke);
        mask_block(s1, key0 + 32, hh, ks, ke);
      }
      float alpha;
      const bool moved = softmax_step(s0, s1, m, l, c, alpha);
      if (!o_zero && wave_ballot(moved)) {
#pragma unroll
        for (int d = 0; d < 4; ++d) o[d] *= alpha;
      }
      o_zero = false;
      // P^T operands: k-step s2 covers keys 16*s2 .. +15 of the tile; lane
      // element t is key 16*s2 + 8*(t>>2) + 4*hh + (t&3).
      bf16x8 pk[4];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pk[0][e] = static_cast<__bf16>(s0[e]);
        pk[1][e] = static_cast<__bf16>(s0[8 + e]);
        pk[2][e] = static_cast<__bf16>(s1[e]);
        pk[3][e] = static_cast<__bf16>(s1[8 + e]);
      }
      // O^T += V^T P^T; the V^T operand is two transposing reads of the same
      // permuted keys (rows 16*s2 + 4*hh + {0..3} and +8).
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        const int r0 = 16 * s2 + vrow;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const char* a = vb + r0 * kRowBytes + ((((4 * d + cq) ^ vsw0)) << 4) + 8 * (i16 & 1);
          const char* a2 =
              vb + (r0 + 8) * kRowBytes + ((((4 * d + cq) ^ vsw1)) << 4) + 8 * (i16 & 1);
          const i16x4 lo = lds_tr16(a);
          const i16x4 hi = lds_tr16(a2);
          const bf16x8 av =
              __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pk[s2], o[d], 0, 0, 0);
        }
      }
    }
    stage = stage == kStages - 1 ? 0 : stage + 1;
  }

  // ---- epilogue: normalise, scatter O rows and log2-LSE ---------------------
  if (valid) {
    const float inv = 1.0f / l;
    uint16_t* orow = p.out + (static_cast<int64_t>(pos) * p.hq + qh) * kD + 4 * hh;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint2 w;
        w.x = pack_bf16x2(o[d][4 * j + 0] * inv, o[d][4 * j + 1] * inv);
        w.y = pack_bf16x2(o[d][4 * j + 2] * inv, o[d][4 * j + 3] * inv);
        *reinterpret_cast<uint2*>(orow + 32 * d + 8 * j) = w;
      }
    }
    if (hh == 0) p.lse[static_cast<int64_t>(pos) * p.hq + qh] = log2f(l) + m * c;
  }
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace
}  // namespace swattn

using namespace swattn;

extern "C" int swattn_prefill_fwd(const void* q, const void* k, const void* v,
                                  const int32_t* full_idx, int64_t n_full,
                                  const int32_t* local_idx, int64_t n_local,
                                  const int32_t* full_starts, const int32_t* local_starts,
                                  const int32_t* causal_ends, void* out, float* lse,
                                  int32_t batch, int64_t seq_q, int64_t seq_kv, int32_t heads_q,
                                  int32_t heads_kv, int32_t head_dim, int32_t window,
                                  float scale_log2, void* stream) {
  if (head_dim != kD) return invalid("swattn_prefill_fwd: head_dim must be 128");
  if (batch < 1 || seq_q < 0 || seq_kv < 1 || heads_q < 1 || heads_kv < 1)
    return invalid("swattn_prefill_fwd: bad shape");
  if (heads_q % heads_kv != 0)
    return invalid("swattn_prefill_fwd: heads_q must be a multiple of heads_kv");
  if (window <= 0) return invalid("swattn_prefill_fwd: window must be positive");
  if (n_full < 0 || n_local < 0 || n_full + n_local > static_cast<int64_t>(batch) * seq_q)
    return invalid("swattn_prefill_fwd: bad index counts");
  const int64_t total_q = static_cast<int64_t>(batch) * seq_q;
  const int64_t total_kv = static_cast<int64_t>(batch) * seq_kv;
  if (total_q > INT32_MAX || total_kv > INT32_MAX - 2 * kBN)
    return invalid("swattn_prefill_fwd: batch*seq must stay below 2^31");
  const int group = heads_q / heads_kv;
  if ((n_full + n_local) * static_cast<int64_t>(group) > INT32_MAX - kRowsPerItem)
    return invalid("swattn_prefill_fwd: too many rows");
  const bool meta = full_starts != nullptr || local_starts != nullptr || causal_ends != nullptr;
  if (meta && (full_starts == nullptr || local_starts == nullptr || causal_ends == nullptr))
    return invalid("swattn_prefill_fwd: metadata needs full_starts, local_starts and causal_ends");
  if (n_full + n_local == 0) return SWATTN_OK;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || lse == nullptr ||
      (n_full > 0 && full_idx == nullptr) || (n_local > 0 && local_idx == nullptr))
    return invalid("swattn_prefill_fwd: null pointer");

  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.out = static_cast<uint16_t*>(out);
  p.lse = lse;
  p.idx[0] = full_idx;
  p.idx[1] = local_idx;
  p.starts[0] = full_starts;
  p.starts[1] = local_starts;
  p.ends = causal_ends;
  p.count[0] = static_cast<int32_t>(n_full);
  p.count[1] = static_cast<int32_t>(n_local);
  p.tiles[0] = static_cast<int32_t>(ceil_div(n_full * group, kRowsPerItem));
  p.tiles[1] = static_cast<int32_t>(ceil_div(n_local * group, kRowsPerItem));
  p.seq_q = static_cast<int32_t>(seq_q);
  p.seq_kv = static_cast<int32_t>(seq_kv);
  p.total_kv = static_cast<int32_t>(total_kv);
  p.hq = heads_q;
  p.hkv = heads_kv;
  p.group = group;
  p.window = window;
  p.c = scale_log2;
  const int64_t grid = (static_cast<int64_t>(p.tiles[0]) + p.tiles[1]) * heads_kv;
  if (grid > INT32_MAX) return invalid("swattn_prefill_fwd: grid too large");
  const hipStream_t st = as_stream(stream);
  if (meta)
    hipLaunchKernelGGL(fwd_kernel<true>, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(fwd_kernel<false>, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, st, p);
  return launch_status("swattn_prefill_fwd");
}
