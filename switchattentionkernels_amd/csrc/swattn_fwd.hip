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
// * Work item = (branch, tile of 128 "rows", KV head).  A row is a
//   (compacted query slot, query head of the KV head's group) pair with the
//   head index fastest, so one K/V tile in LDS serves every query head of the
//   group (GQA packing) and a wave's rows span only 64/G query positions.
// * The whole routed problem is one grid: full-branch tiles first, last tile
//   (longest causal prefix) first, then local tiles; KV head = item % Hkv so
//   that with Hkv = 8 every XCD (blockIdx % 8) streams a single KV head
//   through its own L2.  Counts come from the index lists' lengths, so new
//   routing never recompiles anything.
// * Four waves share each K/V tile; each wave owns 32 rows and computes
//   S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (Q^T stays in registers as the
//   B operand).  Two workgroups per CU put two waves on every SIMD that are
//   not tied by a common barrier, so one wave's softmax (VALU) runs under the
//   other's MFMAs; every accumulator stays in ordinary VGPRs.  Each
//   lane owns one query row and 32 keys of the 64-key tile: row max and row
//   sum are lane-local plus one permlane32 swap.  The S^T accumulator is
//   already the B operand of O^T = V^T P^T once the keys of every 16-key
//   group are permuted consistently on both sides.
// * V is rewritten once per call by vt_pack_kernel into MFMA-ready V^T tiles
//   ([Hkv][key tile][128 d][64 keys], keys permuted, zero-padded): V^T
//   operands are then plain 16-byte LDS reads at the full ds_read_b128 rate
//   (a transposing LDS read of row-major V measured under half that rate).
//   The pre-pass moves 2 x |V| bytes through HBM, a few percent of the
//   attention time.
// * K/V tiles stream global -> LDS with global_load_lds_dwordx4 (no register
//   staging) through a ring of LDS stages, one tile ahead of the compute, with
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

constexpr int kD = 128;                               // head_dim
constexpr int kBN = 64;                               // keys per K/V tile
constexpr int kWaves = 4;                             // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kRowsPerWave = 32;                      // one 32-row MFMA block
constexpr int kRowsPerItem = kWaves * kRowsPerWave;   // 128 rows per work item
constexpr int kRowBytes = kD * 2;                     // 256-byte K rows, unpadded
constexpr int kVtRowBytes = kBN * 2;                  // 128-byte V^T rows (one d, 64 keys)
constexpr int kTileBytes = kBN * kRowBytes;           // one K or V^T tile: 16 KiB
static_assert(kD * kVtRowBytes == kTileBytes, "K and V^T tiles have the same size");
constexpr int kStageBytes = 2 * kTileBytes;           // K + V
constexpr int kStages = 2;                            // LDS ring depth
constexpr int kLdsBytes = kStages * kStageBytes;      // 64 KiB: two workgroups per CU
constexpr int kRowsPerLoader = kBN / kWaves;          // key rows each wave stages per tile
static_assert(kRowsPerLoader % 4 == 0, "a wave stages whole 1 KiB blocks of K and V^T");
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
  const uint16_t* vt;        // packed V^T tiles (vt_pack_kernel)
  int32_t count[2];
  int32_t tiles[2];
  int32_t seq_q, seq_kv, total_kv, kv_tiles;
  int32_t hq, hkv, group, window;
  float c;                   // sm_scale * log2(e)
};

// K chunk swizzle: logical 16-byte chunk j of key row r lives at chunk
// j ^ swz(r).  swz is a permutation of r mod 16, so 16 lanes reading one
// chunk of 16 consecutive rows hit 16 distinct bank groups.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
// V^T chunk swizzle: 128-byte rows pair up in a 256-byte bank line, and
// (d >> 1) & 7 gives the 8 rows of each parity 8 distinct chunks.
__device__ __forceinline__ int vswz(int d) { return (d >> 1) & 7; }
// Position p of a 16-key group of a V^T row holds key perm16(p) of the group:
// the order in which one lane holds P^T elements (lane half h, element t is
// key 8*(t>>2) + 4*h + (t&3), stored at position 8*h + t).
__host__ __device__ constexpr int perm16(int p) {
  return ((p >> 2) & 1) * 8 + (p >> 3) * 4 + (p & 3);
}

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
// 16 bytes per lane from global memory to LDS at lds_base + 16 * lane
// (global_load_lds_dwordx4; the LDS base goes through M0 and must be
// wave-uniform).  Issued as inline assembly so that the compiler's wait
// insertion does not treat it as a store that aliases every LDS read.
// dma16 takes a per-lane 64-bit address; dma16_sbase a wave-uniform base in
// SGPRs plus a per-lane 32-bit byte offset (no per-tile address arithmetic).
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16_sbase(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// Per-lane staging plan for one 64-key tile (constant across tiles): K rows
// and V^T rows go 1 KiB (one lane-linear load) at a time; each wave stages
// kTileBytes / kWaves bytes of each.
// K: load i of wave w writes key rows R*w+4i .. +3 (R = kRowsPerLoader); lane
//    l lands on chunk position l%16 of row l/16 and fetches logical chunk
//    (l%16) ^ swz(row) of that key.
// V^T: load i of wave w writes d rows 2R*w+8i .. +7; lane l lands on chunk
//    position l%8 of row l/8 and fetches logical chunk (l%8) ^ vswz(row).
struct StagePlan {
  uint32_t koff[kRowsPerLoader / 4];   // byte offset of this lane's K chunk from the tile's first key
  uint32_t voff[kRowsPerLoader / 4];   // byte offset of this lane's V^T chunk inside the V^T tile
  int krow[kRowsPerLoader / 4];        // key row inside the tile (for the clamped last tile)
  int kchunk[kRowsPerLoader / 4];
  uint32_t lds_w;                      // this wave's byte offset inside a K (or V^T) tile
};

__device__ __forceinline__ StagePlan make_stage_plan(const FwdParams& p, int kvh, int wave,
                                                     int lane) {
  StagePlan sp;
#pragma unroll
  for (int i = 0; i < kRowsPerLoader / 4; ++i) {
    const int row = kRowsPerLoader * wave + 4 * i + (lane >> 4);
    const int j = (lane & 15) ^ swz(row);
    sp.krow[i] = row;
    sp.kchunk[i] = j;
    sp.koff[i] = static_cast<uint32_t>(((row * p.hkv + kvh) * kD + 8 * j) * 2);
    const int d = 2 * kRowsPerLoader * wave + 8 * i + (lane >> 3);
    const int jv = (lane & 7) ^ vswz(d);
    sp.voff[i] = static_cast<uint32_t>((d * kBN + 8 * jv) * 2);
  }
  sp.lds_w = kRowsPerLoader * wave * kRowBytes;
  return sp;
}

// Issue the loads of tile tk into the stage at LDS byte address stage_lds
// (kLoadsPerTile loads per lane).
__device__ __forceinline__ void stage_tile(const FwdParams& p, const StagePlan& sp,
                                           uint32_t stage_lds, int tk, int kvh) {
  const char* vt_tile = reinterpret_cast<const char*>(p.vt) +
                        (static_cast<int64_t>(kvh) * p.kv_tiles + tk) * kTileBytes;
  const uint32_t lbase = __builtin_amdgcn_readfirstlane(stage_lds + sp.lds_w);
  if ((tk + 1) * kBN <= p.total_kv) {
    const char* k_tile = reinterpret_cast<const char*>(p.k) +
                         static_cast<int64_t>(tk) * kBN * p.hkv * kD * 2;
#pragma unroll
    for (int i = 0; i < kRowsPerLoader / 4; ++i) {
      dma16_sbase(k_tile, sp.koff[i], lbase + 4 * i * kRowBytes);
      dma16_sbase(vt_tile, sp.voff[i], lbase + 4 * i * kRowBytes + kTileBytes);
    }
  } else {
    // Last, partial tile: clamp the key so that every lane reads inside K
    // (the rows past total_kv are masked out of every row's range).
#pragma unroll
    for (int i = 0; i < kRowsPerLoader / 4; ++i) {
      const int key = min(tk * kBN + sp.krow[i], p.total_kv - 1);
      dma16(p.k + (static_cast<int64_t>(key) * p.hkv + kvh) * kD + 8 * sp.kchunk[i],
            lbase + 4 * i * kRowBytes);
      dma16_sbase(vt_tile, sp.voff[i], lbase + 4 * i * kRowBytes + kTileBytes);
    }
  }
}

// V [total_kv, Hkv, 128] -> V^T tiles [Hkv][kv_tiles][128][64]: row d of tile
// t holds V[64t + key][d] for the 64 keys of the tile, each 16-key group in
// perm16 order, zeros past total_kv.  One block per (tile, KV head); the tile
// is staged through LDS (padded rows) and written as coalesced 16-byte chunks.
__global__ __launch_bounds__(256) void vt_pack_kernel(const uint16_t* __restrict__ v,
                                                      uint16_t* __restrict__ vt, int total_kv,
                                                      int hkv, int kv_tiles) {
  __shared__ uint32_t tile[kBN][kD / 2 + 1];   // [key][d pair], odd word stride
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int chunk = tid + 256 * i;           // 64 keys x 16 chunks
    const int key = chunk >> 4, c = chunk & 15;
    const int gk = t * kBN + key;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (gk < total_kv) val = *reinterpret_cast<const uint4*>(v + (static_cast<int64_t>(gk) * hkv + h) * kD + 8 * c);
    tile[key][4 * c + 0] = val.x;
    tile[key][4 * c + 1] = val.y;
    tile[key][4 * c + 2] = val.z;
    tile[key][4 * c + 3] = val.w;
  }
  __syncthreads();
  uint16_t* out = vt + (static_cast<int64_t>(h) * kv_tiles + t) * (kD * kBN);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int chunk = tid + 256 * i;           // 128 d rows x 8 chunks
    const int d = chunk >> 3, c = chunk & 7;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int p0 = 8 * c + 2 * e;
      const int k0 = (p0 & ~15) + perm16(p0 & 15), k1 = (p0 & ~15) + perm16((p0 + 1) & 15);
      const uint32_t lo = (tile[k0][d >> 1] >> (16 * (d & 1))) & 0xffffu;
      const uint32_t hi = (tile[k1][d >> 1] >> (16 * (d & 1))) & 0xffffu;
      w[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(out + d * kBN + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
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

// Mask the keys of a 64-key S^T tile outside [ks, ke).  Register 4j+i of
// block kb holds key offset 32*kb + 8*j + 4*hh + i; lo/hi are the row bounds
// relative to key0 + 4*hh, so each element is one unsigned range test.
__device__ __forceinline__ void mask_tile(f32x16& s0, f32x16& s1, int lo, int hi) {
  const uint32_t span = hi > lo ? static_cast<uint32_t>(hi - lo) : 0u;  // empty row: mask all
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 8 * j + i;
      if (static_cast<uint32_t>(e - lo) >= span) s0[4 * j + i] = -INFINITY;
      if (static_cast<uint32_t>(e + 32 - lo) >= span) s1[4 * j + i] = -INFINITY;
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
  // 32 values -> 16 three-input maxima.
  float mx = fmaxf(fmaxf(s0[0], s0[1]), s0[2]);
#pragma unroll
  for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, s0[e]), s0[e + 1]);
  mx = fmaxf(fmaxf(mx, s0[15]), s1[0]);
#pragma unroll
  for (int e = 1; e < 16; e += 2) mx = fmaxf(fmaxf(mx, s1[e]), s1[e + 1 < 16 ? e + 1 : e]);
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

// Per-wave loop state and per-lane constants.
struct WaveCtx {
  bf16x8 qf[8];        // Q^T B operands
  int koff[8];         // K operand LDS offsets (stage-relative), k-step kk
  int voff[4];         // V^T operand LDS offsets (stage-relative), k-step s2
  int ks, ke;          // this lane's row range
  int w_min_s, w_max_e, w_max_s, w_min_e;
  int hh;
  float c;
  f32x16 o[4];
  float m, l;
  bool o_zero;
};

// One 64-key tile read from LDS stage kStage (compile-time, so every LDS
// address is a per-lane register plus an immediate).
template <int kStage>
__device__ __forceinline__ void tile_step(const FwdParams& p, const StagePlan& sp, char* smem,
                                          int tk, int t_end, int kvh, WaveCtx& w) {
  static_assert(kStages == 2, "tile_step assumes a two-stage ring");
  // This lane's loads of tile tk are complete; after the barrier everyone's
  // are, and every wave has finished reading the other stage, which the
  // loads issued next overwrite.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (tk + 1 < t_end) stage_tile(p, sp, lds_addr(smem) + (kStage ^ 1) * kStageBytes, tk + 1, kvh);
  const int key0 = tk * kBN;
  if (key0 >= w.w_max_e || key0 + kBN <= w.w_min_s) return;  // no row of this wave
  const char* kb = smem + kStage * kStageBytes;
  const char* vb = kb + kTileBytes;
  // S^T = K Q^T: two 32-key blocks.
  f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(kb + w.koff[kk]);
    const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(kb + w.koff[kk] + 32 * kRowBytes);
    s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, w.qf[kk], s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, w.qf[kk], s1, 0, 0, 0);
  }
  if (!(key0 >= w.w_max_s && key0 + kBN <= w.w_min_e))
    mask_tile(s0, s1, w.ks - key0 - 4 * w.hh, w.ke - key0 - 4 * w.hh);
  float alpha;
  const bool moved = softmax_step(s0, s1, w.m, w.l, w.c, alpha);
  if (!w.o_zero && wave_ballot(moved)) {
#pragma unroll
    for (int d = 0; d < 4; ++d) w.o[d] *= alpha;
  }
  w.o_zero = false;
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
  // O^T += V^T P^T, one 16-byte V^T read per MFMA.
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const bf16x8 av = *reinterpret_cast<const bf16x8*>(vb + w.voff[s2] + 32 * d * kVtRowBytes);
      w.o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pk[s2], w.o[d], 0, 0, 0);
    }
  }
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
  WaveCtx w;
  const int r = tile * kRowsPerItem + wave * kRowsPerWave + rl;
  const int slot = r / G;
  const int qh = kvh * G + (r - slot * G);
  const bool valid = slot < count;
  const int pos = idx[valid ? slot : count - 1];
  row_bounds<kMeta>(p, branch, pos, w.ks, w.ke);
  w.hh = hh;
  w.c = p.c;

  // ---- key ranges: wave union / intersection, workgroup union --------------
  w.w_min_s = wave_min(valid ? w.ks : INT_MAX);
  w.w_max_e = wave_max(valid ? w.ke : INT_MIN);
  w.w_max_s = wave_max(valid ? w.ks : INT_MIN);
  w.w_min_e = wave_min(valid ? w.ke : INT_MAX);
  if (lane == 0) {
    s_range[wave] = w.w_min_s;
    s_range[kWaves + wave] = w.w_max_e;
  }
  __syncthreads();
  int g_s = INT_MAX, g_e = INT_MIN;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    g_s = min(g_s, s_range[i]);
    g_e = max(g_e, s_range[kWaves + i]);
  }
  const int t_begin = g_s / kBN;
  const int t_end = g_e > g_s ? (g_e + kBN - 1) / kBN : t_begin;

  // ---- Q row as MFMA B operands (Q^T[d][row]); wait before any LDS load -----
  {
    const uint16_t* qrow = p.q + (static_cast<int64_t>(pos) * p.hq + qh) * kD + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) w.qf[kk] = *reinterpret_cast<const bf16x8*>(qrow + 16 * kk);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- per-lane LDS operand offsets (stage-relative) --------------------------
  // K operand (A of S^T): key row rl (+32 for the second block), logical
  // chunk 2*kk + hh.  V^T operand (A of O^T): d row rl (+32*d), logical chunk
  // 2*s2 + hh, i.e. the 8 permuted keys this lane's P^T elements refer to.
  {
    const int kx = hh ^ swz(rl);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) w.koff[kk] = rl * kRowBytes + (((2 * kk) ^ kx) << 4);
    const int vx = hh ^ vswz(rl);
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) w.voff[s2] = rl * kVtRowBytes + (((2 * s2) ^ vx) << 4);
  }
  const StagePlan sp = make_stage_plan(p, kvh, wave, lane);

#pragma unroll
  for (int d = 0; d < 4; ++d) w.o[d] = f32x16{};
  w.m = kMaxSentinel;
  w.l = 0.f;
  w.o_zero = true;  // O is still exactly zero: a rescale can be skipped

  // ---- main loop: the two-stage ring, unrolled so the stage is static -------
  if (t_begin < t_end) stage_tile(p, sp, lds_addr(smem), t_begin, kvh);
  for (int tk = t_begin; tk < t_end; tk += 2) {
    tile_step<0>(p, sp, smem, tk, t_end, kvh, w);
    if (tk + 1 < t_end) tile_step<1>(p, sp, smem, tk + 1, t_end, kvh, w);
  }

  // ---- epilogue: normalise, scatter O rows and log2-LSE ---------------------
  if (valid) {
    const float inv = 1.0f / w.l;
    uint16_t* orow = p.out + (static_cast<int64_t>(pos) * p.hq + qh) * kD + 4 * hh;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint2 u;
        u.x = pack_bf16x2(w.o[d][4 * j + 0] * inv, w.o[d][4 * j + 1] * inv);
        u.y = pack_bf16x2(w.o[d][4 * j + 2] * inv, w.o[d][4 * j + 3] * inv);
        *reinterpret_cast<uint2*>(orow + 32 * d + 8 * j) = u;
      }
    }
    if (hh == 0) p.lse[static_cast<int64_t>(pos) * p.hq + qh] = log2f(w.l) + w.m * w.c;
  }
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace
}  // namespace swattn

using namespace swattn;

inline int64_t kv_tiles_for(int64_t total_kv) { return ceil_div(total_kv, kBN); }

extern "C" size_t swattn_prefill_workspace_bytes(int32_t batch, int64_t seq_kv, int32_t heads_kv,
                                                 int32_t head_dim) {
  if (batch < 1 || seq_kv < 1 || heads_kv < 1 || head_dim != kD) return 0;
  return static_cast<size_t>(heads_kv) * kv_tiles_for(static_cast<int64_t>(batch) * seq_kv) *
         kTileBytes;
}

extern "C" int swattn_prefill_fwd(const void* q, const void* k, const void* v,
                                  const int32_t* full_idx, int64_t n_full,
                                  const int32_t* local_idx, int64_t n_local,
                                  const int32_t* full_starts, const int32_t* local_starts,
                                  const int32_t* causal_ends, void* out, float* lse,
                                  int32_t batch, int64_t seq_q, int64_t seq_kv, int32_t heads_q,
                                  int32_t heads_kv, int32_t head_dim, int32_t window,
                                  float scale_log2, void* workspace, size_t workspace_bytes,
                                  void* stream) {
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
  const size_t ws_need = swattn_prefill_workspace_bytes(batch, seq_kv, heads_kv, head_dim);
  if (workspace == nullptr || workspace_bytes < ws_need) {
    set_error("swattn_prefill_fwd: workspace smaller than swattn_prefill_workspace_bytes()");
    return SWATTN_EWORKSPACE;
  }

  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.vt = static_cast<const uint16_t*>(workspace);
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
  p.kv_tiles = static_cast<int32_t>(kv_tiles_for(total_kv));
  p.hq = heads_q;
  p.hkv = heads_kv;
  p.group = group;
  p.window = window;
  p.c = scale_log2;
  const int64_t grid = (static_cast<int64_t>(p.tiles[0]) + p.tiles[1]) * heads_kv;
  if (grid > INT32_MAX) return invalid("swattn_prefill_fwd: grid too large");
  const hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(vt_pack_kernel, dim3(p.kv_tiles, heads_kv), dim3(256), 0, st, p.v,
                     static_cast<uint16_t*>(workspace), p.total_kv, heads_kv, p.kv_tiles);
  if (meta)
    hipLaunchKernelGGL(fwd_kernel<true>, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(fwd_kernel<false>, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, st, p);
  return launch_status("swattn_prefill_fwd");
}
