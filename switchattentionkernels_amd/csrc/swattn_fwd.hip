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
//   group (GQA packing) and a wave's 32 rows span only 32/G query positions.
// * The whole routed problem is one grid: full-branch tiles first, then
//   local tiles, each branch from its last tile (latest positions) down, so
//   that work items come roughly longest first; KV head = item % Hkv so
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
// * K/V^T tiles stream global -> LDS with buffer_load_dwordx4 ... lds (no
//   register staging) into a two-slot K ring and a two-slot V^T ring, with
//   one barrier per tile.  The buffer descriptor's range check stops a tile
//   at the end of the sequence, so there is no clamped slow path and no
//   branch around the loads.  The loads are issued from inline assembly and
//   waited for with explicit vmcnt counts: the compiler cannot see that they
//   target another slot than the one being read, and would otherwise drain
//   every load before each LDS read.  LDS rows are unpadded 256-byte rows
//   whose 16-byte chunks are XOR-swizzled so both operand read patterns are
//   conflict-free.
// * The tile loop is software-pipelined inside each wave: while the matrix
//   cores compute S for tile j+1, the VALU turns S(j) into P(j); while they
//   accumulate P(j) V(j), the VALU sums P(j) and takes the max of S(j+1).
//   K therefore runs one tile ahead of V^T.  Each phase is one basic block
//   with an explicit MFMA/VALU/LDS-read interleave.
// * The running max is only moved when it grows by more than 2^8 in the
//   exp2 domain (rescaling O is then rare); P = 2^(s*c - m*c) stays below
//   2^8, and O = acc / l, LSE = log2(l) + m*c are the same quantities as with
//   an exact running max.
// * Tiles outside a wave's key range are skipped and interior tiles skip the
//   mask.
// * Key-range split (fwd_kernel<., true>, host plan in split_plan): when the
//   longest causal item is long against the rest of the work (few KV heads,
//   e.g. one GPU's share of a KV-head split, or short sequences on few
//   heads), each full item runs as one workgroup per chunk of its range
//   (4 to 64 key tiles planned per call, longer for very long sequences so
//   that the chunk slots stay near 2048).  The chunks' fp32 O rows and
//   LSE go to the workspace and fwd_merge_kernel folds them (log2 LSE,
//   V:236-241).  Chunk boundaries are fixed multiples of the chunk size,
//   and an item inside one chunk is computed exactly as without a split.

#include <limits.h>
#include <math.h>

#include <algorithm>

#include "tiles.h"

namespace swattn {
namespace {

using namespace tiles;

#ifndef SWATTN_WAVES
#define SWATTN_WAVES 4
#endif
constexpr int kWaves = SWATTN_WAVES;                  // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kRowsPerWave = 32;                      // one 32-row MFMA block
constexpr int kRowsPerItem = kWaves * kRowsPerWave;   // 128 rows per work item
// LDS: a two-slot K ring followed by a two-slot V^T ring (K runs one tile
// ahead of V^T).  64 KiB: two workgroups per CU.
constexpr int kVRing = 2 * kTileBytes;                // byte offset of the V^T ring
constexpr int kLdsBytes = 4 * kTileBytes;
constexpr int kRowsPerLoader = kBN / kWaves;          // key rows each wave stages per tile
static_assert(kRowsPerLoader % 4 == 0, "a wave stages whole 1 KiB blocks of K and V^T");
constexpr int kLoads = kRowsPerLoader / 4;            // loads per lane per K (or V^T) tile
static_assert(kLoads == 1 || kLoads == 2 || kLoads == 4, "loads spread over 8 / 4 k-steps");
constexpr float kMaxSentinel = -1073741824.0f;        // -2^30 (V:174)
// The rings, or the O epilogue's staging if that is larger (eight waves).
constexpr int kSmemBytes = kLdsBytes > kWaves * kStoreRegionBytes ? kLdsBytes
                                                                   : kWaves * kStoreRegionBytes;

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
  int32_t seq_q, seq_kv, total_q, total_kv, kv_tiles;
  int32_t hq, hkv, group, window;
  float c;                   // sm_scale * log2(e)
  // Key-range split of full items (maxc > 1): a full item whose key tiles
  // cross a multiple of split_tiles runs as one workgroup per such chunk.
  int32_t maxc;              // chunk slots per full item (1: no split)
  int32_t split_tiles;       // chunk size in 64-key tiles (maxc > 1)
  float* part_o;             // [full item][slot][128 rows][128] fp32 O of the chunk (normalised)
  float* part_lse;           // [full item][slot][128 rows] log2 LSE of the chunk (-inf: no key)
  int2* part_n;              // [full item] (chunks, first chunk); chunks > 1: merge needed
};

// Chunk of the key-range split, in 64-key tiles: between kSplitMinTiles and
// kSplitTiles (4096 keys), chosen per call, and longer for very long
// sequences (split_plan keeps the chunk slots near kSplitMaxChunks).  Boundaries sit at fixed
// multiples of it, so a row's chunks depend only on its own range, and an
// item inside one chunk is computed exactly as without a split.
constexpr int kSplitTiles = 64;
constexpr int kSplitMinTiles = 4;

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
  uint32_t lds_w;                      // this wave's byte offset inside a K (or V^T) tile
};

__device__ __forceinline__ StagePlan make_stage_plan(const FwdParams& p, int kvh, int wave,
                                                     int lane) {
  StagePlan sp;
#pragma unroll
  for (int i = 0; i < kRowsPerLoader / 4; ++i) {
    const int row = kRowsPerLoader * wave + 4 * i + (lane >> 4);
    const int j = (lane & 15) ^ swz(row);
    sp.koff[i] = static_cast<uint32_t>(((row * p.hkv + kvh) * kD + 8 * j) * 2);
    const int d = 2 * kRowsPerLoader * wave + 8 * i + (lane >> 3);
    const int jv = (lane & 7) ^ vswz(d);
    sp.voff[i] = static_cast<uint32_t>((d * kBN + 8 * jv) * 2);
  }
  sp.lds_w = kRowsPerLoader * wave * kRowBytes;
  return sp;
}

// Buffer descriptor for K tile tk of KV head kvh (any lane offset of the
// staging plan); rows past total_kv fall outside it.  `live` = false gives an
// empty descriptor: the step's K loads then move nothing.
__device__ __forceinline__ i32x4 k_rsrc(const FwdParams& p, int tk, bool live) {
  const int64_t row_bytes = static_cast<int64_t>(p.hkv) * kD * 2;
  const int t = live ? tk : 0;
  const int64_t rest = (static_cast<int64_t>(p.total_kv) - static_cast<int64_t>(t) * kBN) * row_bytes;
  const uint32_t n = live ? static_cast<uint32_t>(rest < 0xffffffffLL ? rest : 0xffffffffLL) : 0u;
  return make_rsrc(reinterpret_cast<const char*>(p.k) + static_cast<int64_t>(t) * kBN * row_bytes, n);
}

// Buffer descriptor for V^T tile tk of KV head kvh (zero-padded, always whole).
__device__ __forceinline__ i32x4 v_rsrc(const FwdParams& p, int tk, int kvh, bool live) {
  const int t = live ? tk : 0;
  return make_rsrc(reinterpret_cast<const char*>(p.vt) +
                       (static_cast<int64_t>(kvh) * p.kv_tiles + t) * kTileBytes,
                   live ? static_cast<uint32_t>(kTileBytes) : 0u);
}

// Load i (of kRowsPerLoader / 4) of this wave's share of a K or V^T tile
// into the slot at LDS byte address slot.
__device__ __forceinline__ void stage_k(const StagePlan& sp, const i32x4& rs, uint32_t slot, int i) {
  dma16(rs, sp.koff[i], __builtin_amdgcn_readfirstlane(slot + sp.lds_w + 4 * i * kRowBytes));
}
__device__ __forceinline__ void stage_v(const StagePlan& sp, const i32x4& rs, uint32_t slot, int i) {
  dma16(rs, sp.voff[i], __builtin_amdgcn_readfirstlane(slot + sp.lds_w + 4 * i * kRowBytes));
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

// Row max of a 32-row x 64-key tile held as two S^T blocks: 32 values per
// lane in 16 three-input maxima, then the other half-wave's 32 keys.
__device__ __forceinline__ float tile_max(const f32x16& s0, const f32x16& s1) {
  float mx = fmaxf(fmaxf(s0[0], s0[1]), s0[2]);
#pragma unroll
  for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, s0[e]), s0[e + 1]);
  mx = fmaxf(fmaxf(mx, s0[15]), s1[0]);
#pragma unroll
  for (int e = 1; e < 16; e += 2) mx = fmaxf(fmaxf(mx, s1[e]), s1[e + 1 < 16 ? e + 1 : e]);
  return xor32_max(mx);
}

// P = 2^(s*c - m*c) in place.
__device__ __forceinline__ void tile_exp(f32x16& s0, f32x16& s1, float c, float mc) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    s0[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[e], c, -mc));
    s1[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[e], c, -mc));
  }
}

// Row sum of the fp32 P tile (both half-waves).
__device__ __forceinline__ float tile_sum(const f32x16& s0, const f32x16& s1) {
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    a += s0[e];
    b += s1[e];
  }
  return xor32_sum(a + b);
}

// Per-wave loop state and per-lane constants.
struct WaveCtx {
  bf16x8 qf[8];        // Q^T B operands
  int koff[8];         // K operand LDS offsets (slot-relative), k-step kk
  int voff[4];         // V^T operand LDS offsets (slot-relative), k-step s2
  int ks, ke;          // this lane's row range
  int w_min_s, w_max_e, w_max_s, w_min_e;
  int it0, it1;        // tiles inside every row's range (no mask): [it0, it1)
  int hh;
  float c;
  f32x16 o[4];
  float m, l;
  float alpha;         // O / l rescale factor of the last tile whose max was taken
  bool rescale;        // some lane's max moved at that tile
  bool o_zero;
};

__device__ __forceinline__ bool wave_has_keys(const WaveCtx& w, int tk) {
  const int key0 = tk * kBN;
  return key0 < w.w_max_e && key0 + kBN > w.w_min_s;
}

// S^T = K Q^T for the K tile at kb: two 32-key blocks, one 16-byte K read per
// MFMA.  The step's K staging loads (into another slot) are spread over the
// tile, one after every second pair of reads.
__device__ __forceinline__ void qk_tile(const char* kb, const WaveCtx& w, f32x16& s0, f32x16& s1,
                                        const StagePlan& sp, const i32x4& krs, uint32_t kslot) {
  s0 = f32x16{};
  s1 = f32x16{};
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(kb + w.koff[kk]);
    const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(kb + w.koff[kk] + 32 * kRowBytes);
    if ((kk + 1) % (8 / kLoads) == 0) stage_k(sp, krs, kslot, kk / (8 / kLoads));
    s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, w.qf[kk], s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, w.qf[kk], s1, 0, 0, 0);
  }
}

// P^T as bf16 MFMA B operands: k-step s2 covers keys 16*s2 .. +15 of the
// tile; lane element t is key 16*s2 + 8*(t>>2) + 4*hh + (t&3).
__device__ __forceinline__ void pack_p(const f32x16& p0, const f32x16& p1, bf16x8 (&pk)[4]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pk[0][e] = static_cast<__bf16>(p0[e]);
    pk[1][e] = static_cast<__bf16>(p0[8 + e]);
    pk[2][e] = static_cast<__bf16>(p1[e]);
    pk[3][e] = static_cast<__bf16>(p1[8 + e]);
  }
}

// O^T += V^T P^T for the V^T tile at vb, one 16-byte V^T read per MFMA; the
// step's V^T staging loads are spread over the tile, one per k-step.
__device__ __forceinline__ void pv_tile(const char* vb, WaveCtx& w, const bf16x8 (&pk)[4],
                                        const StagePlan& sp, const i32x4& vrs, uint32_t vslot) {
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const bf16x8 av = *reinterpret_cast<const bf16x8*>(vb + w.voff[s2] + 32 * d * kVtRowBytes);
      w.o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pk[s2], w.o[d], 0, 0, 0);
    }
    if ((s2 + 1) % (4 / kLoads) == 0) stage_v(sp, vrs, vslot, s2 / (4 / kLoads));
  }
}

// Take the max of the (masked) S tile n0/n1 into the running max.  m only
// moves when the tile max exceeds it by more than 8 in the exp2 domain (or m
// is still the sentinel); alpha is then the rescale factor for O and l,
// otherwise exactly 1.
__device__ __forceinline__ void take_max(const f32x16& n0, const f32x16& n1, WaveCtx& w) {
  const float mx = tile_max(n0, n1);
  const bool moved = (mx - w.m) * w.c > 8.0f;
  const float m_new = moved ? mx : w.m;
  w.alpha = moved ? __builtin_amdgcn_exp2f((w.m - m_new) * w.c) : 1.0f;
  w.rescale = wave_ballot(moved) != 0;
  w.m = m_new;
}

// Scheduling pattern for a region holding 16 MFMAs, their 16 LDS operand
// reads and independent VALU work: three reads up front, then each MFMA is
// followed by kValu VALU instructions and the next read (three reads in
// flight measured 1 % faster than two, four no better than three).
// Instruction masks: 0x008 MFMA, 0x002 VALU, 0x100 LDS read.
#ifndef SWATTN_LDS_AHEAD
#define SWATTN_LDS_AHEAD 3
#endif
template <int kValu>
__device__ __forceinline__ void interleave_16_mfma() {
  constexpr int kAhead = SWATTN_LDS_AHEAD;   // operand reads issued before the first MFMA
  __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
    if (i < 16 - kAhead) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
}

// One pipeline step, for tile j = t_begin + r:
//   phase A: S(j+1) = K(j+1) Q^T on the matrix cores while the VALU turns
//            S(j) into P(j) (m, taken in the previous step, is final for j);
//   between: the (rare) O rescale for tile j and the mask of S(j+1);
//   phase B: O += V(j) P(j) on the matrix cores while the VALU sums P(j)
//            and takes the max of S(j+1).
// The two phases are single basic blocks, so the compiler interleaves the
// independent MFMA and VALU streams.  kPar = r & 1 selects the LDS slots
// (K read kPar^1, V^T read kPar) and the S buffers (current sb[kPar], next
// sb[kPar^1]) at compile time.  Every wave stages its share of K(j+2) into
// K slot kPar during phase A and of V^T(j+1) into V^T slot kPar^1 during
// phase B, whatever it computes itself.
template <int kPar, bool kS, bool kPV>
__device__ __forceinline__ void pipe_body(const char* smem, const StagePlan& sp, const i32x4& krs,
                                          const i32x4& vrs, int j, WaveCtx& w,
                                          f32x16 (&sb)[2][2]) {
  const char* kb = smem + (kPar ^ 1) * kTileBytes;
  const char* vb = smem + kVRing + kPar * kTileBytes;
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t kslot = lds0 + kPar * kTileBytes;
  const uint32_t vslot = lds0 + kVRing + (kPar ^ 1) * kTileBytes;
  f32x16& c0 = sb[kPar][0];
  f32x16& c1 = sb[kPar][1];
  f32x16& n0 = sb[kPar ^ 1][0];
  f32x16& n1 = sb[kPar ^ 1][1];
  // phase A.  In a full step the wave issues at raised priority during phase
  // A (the exponentials) and at normal priority during phase B: where the two
  // waves of a SIMD compete, phase A goes first (0.4-0.9 % faster at p_full
  // 0.25-1 than no priorities, bit-identical).
  bf16x8 pk[4];
  if constexpr (kS && kPV) __builtin_amdgcn_s_setprio(1);
  if constexpr (kS) {
    qk_tile(kb, w, n0, n1, sp, krs, kslot);
  } else {
#pragma unroll
    for (int i = 0; i < kRowsPerLoader / 4; ++i) stage_k(sp, krs, kslot, i);
  }
  if constexpr (kPV) {
    tile_exp(c0, c1, w.c, w.m * w.c);
    pack_p(c0, c1, pk);
    if constexpr (kS) interleave_16_mfma<5>();   // 32 fma + 32 exp + 16 cvt
    // Materialise P here: without this the compiler sinks the exponentials
    // past the branches below into phase B, next to their only MFMA users,
    // and phase A is left with no VALU work to hide under its MFMAs.
    asm volatile("" : "+v"(c0), "+v"(c1), "+v"(pk[0]), "+v"(pk[1]), "+v"(pk[2]), "+v"(pk[3]));
  }
  // between the phases
  if constexpr (kPV) {
    if (w.rescale && !w.o_zero) {
#pragma unroll
      for (int d = 0; d < 4; ++d) w.o[d] *= w.alpha;
    }
    w.o_zero = false;
  }
  if constexpr (kS) {
    if (j + 1 < w.it0 || j + 1 >= w.it1) {
      const int key0 = (j + 1) * kBN;
      mask_tile(n0, n1, w.ks - key0 - 4 * w.hh, w.ke - key0 - 4 * w.hh);
    }
  }
  // phase B
  if constexpr (kS && kPV) __builtin_amdgcn_s_setprio(0);
  if constexpr (kPV) {
    pv_tile(vb, w, pk, sp, vrs, vslot);
    w.l = w.l * w.alpha + tile_sum(c0, c1);
  } else {
#pragma unroll
    for (int i = 0; i < kRowsPerLoader / 4; ++i) stage_v(sp, vrs, vslot, i);
  }
  if constexpr (kS) take_max(n0, n1, w);
  if constexpr (kS && kPV) interleave_16_mfma<4>();   // row sum + row max, ~65 VALU
}

template <int kPar>
__device__ __forceinline__ void pipe_step(const FwdParams& p, const StagePlan& sp, char* smem,
                                          int r, int t_begin, int n_tiles, int kvh, WaveCtx& w,
                                          f32x16 (&sb)[2][2]) {
  // Every lane's loads of K(j+1) and V(j) are complete after the barrier, and
  // every wave has finished step r-1, which read the K slot and the V^T slot
  // that this step's loads overwrite.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const int j = t_begin + r;
  const i32x4 krs = k_rsrc(p, j + 2, r + 2 < n_tiles);
  const i32x4 vrs = v_rsrc(p, j + 1, kvh, r + 1 < n_tiles);
  const bool do_s = r + 1 < n_tiles && wave_has_keys(w, j + 1);
  const bool do_pv = r >= 0 && wave_has_keys(w, j);
  if (do_s && do_pv)
    pipe_body<kPar, true, true>(smem, sp, krs, vrs, j, w, sb);
  else if (do_s)
    pipe_body<kPar, true, false>(smem, sp, krs, vrs, j, w, sb);
  else if (do_pv)
    pipe_body<kPar, false, true>(smem, sp, krs, vrs, j, w, sb);
  else
    pipe_body<kPar, false, false>(smem, sp, krs, vrs, j, w, sb);
}

// kSplit: the grid holds p.maxc chunk slots per full item (key-range split);
// without it, the kernel has none of the split's code.
template <bool kMeta, bool kSplit>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(2, 2))) void fwd_kernel(const FwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kSmemBytes];
  __shared__ int s_range[2 * kWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rl = lane & 31, hh = lane >> 5;

  // ---- work item -> (branch, tile, chunk slot, kv head) ----------------------
  // Full tiles come first, each as maxc chunk slots in a row; KV head fastest.
  const int item = blockIdx.x;
  const int kvh = item % p.hkv;
  const int tq = item / p.hkv;
  const int full_slots = kSplit ? p.tiles[0] * p.maxc : p.tiles[0];
  const int t = !kSplit ? tq : tq < full_slots ? tq / p.maxc : p.tiles[0] + (tq - full_slots);
  const int cslot = kSplit && tq < full_slots ? tq - t * p.maxc : 0;
  const int branch = t < p.tiles[0] ? 0 : 1;
  // Both branches run their last tile (latest positions) first: full tiles
  // are then ordered by falling causal length, and the local tiles that end
  // the grid are the short ones whose window is cut at the sequence start.
  const int tile = branch == 0 ? p.tiles[0] - 1 - t : p.tiles[0] + p.tiles[1] - 1 - t;
  const int32_t* __restrict__ idx = p.idx[branch];
  const int count = p.count[branch];
  const int G = p.group;

  // ---- this lane's row ------------------------------------------------------
  WaveCtx w;
  const int r = tile * kRowsPerItem + wave * kRowsPerWave + rl;
  const int slot = r / G;
  const int qh = kvh * G + (r - slot * G);
  // A listed position outside [0, total_q) is treated like a padding row:
  // nothing is read at it and nothing is stored for it.  The host checks the
  // lists before the launch; this keeps a list changed after that check from
  // turning into an out-of-bounds access.
  const int listed = idx[slot < count ? slot : count - 1];
  const bool in_range = static_cast<uint32_t>(listed) < static_cast<uint32_t>(p.total_q);
  const bool valid = slot < count && in_range;
  const int pos = in_range ? listed : 0;
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
  int t_begin = g_s / kBN;
  int t_end = g_e > g_s ? (g_e + kBN - 1) / kBN : t_begin;
  // Key-range split: chunk slot k of a full item is chunk c0 + k of its
  // tiles; slots past its last chunk do nothing.  An item whose rows span
  // more chunks than it has slots (a sparse list over several sequences) runs
  // whole in slot 0.  Every full item records (chunks, c0) once, from slot
  // 0, for the merge (chunks 1: nothing to merge).
  bool split_item = false;
  if (kSplit && branch == 0) {
    const int c0 = t_end > t_begin ? t_begin / p.split_tiles : 0;
    const int c1 = t_end > t_begin ? (t_end - 1) / p.split_tiles : 0;
    const int nch = c1 - c0 + 1 <= p.maxc ? c1 - c0 + 1 : 1;
    if (cslot >= nch) return;   // uniform: every wave has the same range
    split_item = nch > 1;
    if (cslot == 0 && tid == 0) p.part_n[t * p.hkv + kvh] = make_int2(nch, c0);
    if (split_item) {
      const int c = c0 + cslot;
      t_begin = max(t_begin, c * p.split_tiles);
      t_end = min(t_end, (c + 1) * p.split_tiles);
    }
  }
  // Tiles inside every row's range (they skip the mask), as scalars.  (The
  // tile-skip test stays on vector registers: as a scalar condition it lets
  // the compiler restructure the step so that its registers overflow.)
  {
    const int ms = __builtin_amdgcn_readfirstlane(w.w_max_s);
    const int me = __builtin_amdgcn_readfirstlane(w.w_min_e);
    w.it0 = (ms + kBN - 1) / kBN;          // first tile with key0 >= every row start
    w.it1 = me > 0 ? me / kBN : 0;         // tiles with key0 + 64 <= every row end
  }

  // ---- Q row as MFMA B operands (Q^T[d][row]); wait before any LDS load -----
  {
    const uint16_t* qrow = p.q + (static_cast<int64_t>(pos) * p.hq + qh) * kD + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) w.qf[kk] = *reinterpret_cast<const bf16x8*>(qrow + 16 * kk);
  }
  // Wait for the Q loads with the builtin, not inline assembly: the compiler
  // then knows they are complete.  Otherwise it keeps them "outstanding"
  // into the tile loop and, at their first use there, emits vmcnt waits that
  // also drain the next tile's LDS loads issued by then.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

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
  w.alpha = 1.f;
  w.rescale = false;
  w.o_zero = true;  // O is still exactly zero: a rescale can be skipped

  // ---- main loop: step r computes S(t_begin+r+1) and O += V P(t_begin+r) -----
  // Unrolled by two so that LDS slots and S buffers are static; step -1 only
  // computes the first S tile.
  const int n_tiles = t_end - t_begin;
  f32x16 sb[2][2];
  {
    const i32x4 krs = k_rsrc(p, t_begin, n_tiles > 0);
#pragma unroll
    for (int i = 0; i < kRowsPerLoader / 4; ++i) stage_k(sp, krs, lds_addr(smem), i);
  }
  for (int r = -1; r < n_tiles; r += 2) {
    pipe_step<1>(p, sp, smem, r, t_begin, n_tiles, kvh, w, sb);
    if (r + 1 < n_tiles) pipe_step<0>(p, sp, smem, r + 1, t_begin, n_tiles, kvh, w, sb);
  }

  // ---- epilogue: normalise, write O rows and log2-LSE -------------------------
  // O goes out as whole rows through LDS (store_rows_via_lds).  The rings are
  // free once every wave's last loads (empty descriptors) have landed and
  // every wave is past its last tile.
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  if (kSplit && split_item) {
    // One chunk of a split item: its normalised fp32 O rows and log2 LSE
    // (a row with no key in the chunk: O 0, LSE -inf); fwd_merge_kernel
    // folds the chunks.  Element 4j+e of accumulator d is d-row
    // 32d + 8j + 4hh + e of this lane's row.
    const int64_t ps = static_cast<int64_t>(t * p.hkv + kvh) * p.maxc + cslot;
    const int rr = wave * kRowsPerWave + rl;
    const float inv = w.l > 0.f ? 1.0f / w.l : 0.f;
    float* po = p.part_o + (ps * kRowsPerItem + rr) * kD + 4 * hh;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<float4*>(po + 32 * d + 8 * j) =
            make_float4(w.o[d][4 * j] * inv, w.o[d][4 * j + 1] * inv, w.o[d][4 * j + 2] * inv,
                        w.o[d][4 * j + 3] * inv);
    }
    if (hh == 0)
      p.part_lse[ps * kRowsPerItem + rr] = w.l > 0.f ? log2f(w.l) + w.m * w.c : -INFINITY;
    return;
  }
  if (valid && hh == 0) p.lse[static_cast<int64_t>(pos) * p.hq + qh] = log2f(w.l) + w.m * w.c;
  store_rows_via_lds(smem + wave * kStoreRegionBytes,
                     valid ? (static_cast<int64_t>(pos) * p.hq + qh) * kD : -1, w.o, 1.0f / w.l,
                     p.out, lane);
}

// Rows of split full items: O = sum_c 2^(LSE_c - LSE) O_c and LSE = log2
// sum_c 2^LSE_c over the item's chunks (those with LSE_c = -inf skipped; a
// row with no key in any chunk is 0 / 0 = NaN with LSE -inf, as the unsplit
// kernel writes it).  One thread per (full item, row, 4 of the 128 d), the
// chunks summed in order.
__global__ __launch_bounds__(256) void fwd_merge_kernel(const FwdParams p) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int q4 = static_cast<int>(id & 31);
  const int rr = static_cast<int>((id >> 5) & (kRowsPerItem - 1));
  const int fi = static_cast<int>(id >> 12);   // full item = t * hkv + kvh
  if (fi >= p.tiles[0] * p.hkv) return;
  const int2 nc = p.part_n[fi];
  if (nc.x <= 1) return;   // computed whole by its workgroup
  const int t = fi / p.hkv, kvh = fi - t * p.hkv;
  const int tile = p.tiles[0] - 1 - t;
  const int r = tile * kRowsPerItem + rr;
  const int G = p.group;
  const int slot = r / G;
  if (slot >= p.count[0]) return;
  const int listed = p.idx[0][slot];
  if (static_cast<uint32_t>(listed) >= static_cast<uint32_t>(p.total_q)) return;
  const int qh = kvh * G + (r - slot * G);
  const int64_t ps0 = static_cast<int64_t>(fi) * p.maxc;
  float mx = -INFINITY;
  for (int k = 0; k < nc.x; ++k) mx = fmaxf(mx, p.part_lse[(ps0 + k) * kRowsPerItem + rr]);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float lsum = 0.f;
  if (mx != -INFINITY) {
    for (int k = 0; k < nc.x; ++k) {
      const float lc = p.part_lse[(ps0 + k) * kRowsPerItem + rr];
      if (lc == -INFINITY) continue;
      const float wgt = exp2f(lc - mx);
      const float4 o = reinterpret_cast<const float4*>(
          p.part_o + ((ps0 + k) * kRowsPerItem + rr) * kD)[q4];
      acc.x += wgt * o.x;
      acc.y += wgt * o.y;
      acc.z += wgt * o.z;
      acc.w += wgt * o.w;
      lsum += wgt;
    }
  }
  const float inv = 1.0f / lsum;   // no key at all: 0 / 0 = NaN
  uint2 u;
  u.x = pack_bf16x2(acc.x * inv, acc.y * inv);
  u.y = pack_bf16x2(acc.z * inv, acc.w * inv);
  const int64_t row = static_cast<int64_t>(listed) * p.hq + qh;
  *reinterpret_cast<uint2*>(p.out + row * kD + 4 * q4) = u;
  if (q4 == 0) p.lse[row] = mx == -INFINITY ? -INFINITY : mx + log2f(lsum);
}

}  // namespace
}  // namespace swattn

using namespace swattn;
using namespace swattn::tiles;

inline int64_t kv_tiles_for(int64_t total_kv) { return ceil_div(total_kv, kBN); }
inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Key-range split plan.  A full item spans up to ceil(seq_kv / 64) + 1 key
// tiles; when that is more than twice the estimated tiles per workgroup slot
// (two per CU of a 256-CU MI355X), one long causal item would set the
// kernel's length, so full items are split into chunks of 1.5 times that
// estimate, clamped to [kSplitMinTiles, kSplitTiles], if the longest spans
// more than one and a half chunks.  (Same-box A/B on eleven shapes against
// chunks of twice the estimate capped at 32 tiles: 5-25 % faster on four
// few-head shapes, within 3 % on the rest, the large-grid configurations
// unsplit either way.)  The estimate counts full items at half a sequence
// of tiles and local items at their window.  Workspace after the V^T tiles:
// the chunks' fp32 O rows, their LSE and one (chunks, first chunk) per full
// item.
constexpr int64_t kSplitSlots = 512;
constexpr int64_t kSplitMaxChunks = 2048;
struct SplitPlan {
  int32_t maxc = 1;
  int32_t tiles = kSplitTiles;
  size_t off_o = 0, off_lse = 0, off_n = 0, bytes = 0;   // offsets from the workspace start
};

inline SplitPlan split_plan(int32_t batch, int64_t seq_kv, int32_t heads_q, int32_t heads_kv,
                            int32_t window, int64_t n_full, int64_t n_local) {
  SplitPlan sp;
  const int64_t group = heads_q / heads_kv;
  const int64_t full_items = ceil_div(n_full * group, kRowsPerItem);
  const int64_t local_items = ceil_div(n_local * group, kRowsPerItem);
  const int64_t seq_tiles = ceil_div(seq_kv, kBN);
  const int64_t longest = full_items > 0 ? seq_tiles + 1 : 0;
  const int64_t local_tiles = ceil_div(std::min<int64_t>(window, seq_kv), kBN) + 2;
  const int64_t est = heads_kv * (full_items * (seq_tiles / 2 + 2) + local_items * local_tiles);
  const int64_t per_slot = est / kSplitSlots;
  int64_t chunk = std::min<int64_t>(kSplitTiles, std::max<int64_t>(kSplitMinTiles, (3 * per_slot) / 2));
  // Very long sequences: chunks long enough that the chunk slots number at
  // most about kSplitMaxChunks.  With the split condition below, full items
  // times KV heads stay under 512, so the slots stay under kSplitMaxChunks +
  // 1024 and their fp32 rows under 200 MiB.
  chunk = std::max<int64_t>(chunk, ceil_div(full_items * heads_kv * seq_tiles, kSplitMaxChunks));
  if (2 * longest <= 3 * chunk || longest <= 2 * per_slot) return sp;
  sp.tiles = static_cast<int32_t>(chunk);
  sp.maxc = static_cast<int32_t>(ceil_div(seq_tiles, chunk) + 1);
  const size_t slots = static_cast<size_t>(full_items * heads_kv) * sp.maxc;
  size_t o = align256(static_cast<size_t>(heads_kv) * kv_tiles_for(static_cast<int64_t>(batch) * seq_kv) *
                      kTileBytes);
  sp.off_o = o;   o = align256(o + slots * kRowsPerItem * kD * sizeof(float));
  sp.off_lse = o; o = align256(o + slots * kRowsPerItem * sizeof(float));
  sp.off_n = o;   o = align256(o + static_cast<size_t>(full_items * heads_kv) * sizeof(int2));
  sp.bytes = o;
  return sp;
}

extern "C" size_t swattn_prefill_workspace_bytes(int32_t batch, int64_t seq_kv, int32_t heads_kv,
                                                 int32_t head_dim) {
  if (batch < 1 || seq_kv < 1 || heads_kv < 1 || head_dim != kD) return 0;
  return static_cast<size_t>(heads_kv) * kv_tiles_for(static_cast<int64_t>(batch) * seq_kv) *
         kTileBytes;
}

extern "C" size_t swattn_prefill_split_workspace_bytes(int32_t batch, int64_t seq_q,
                                                       int64_t seq_kv, int32_t heads_q,
                                                       int32_t heads_kv, int32_t head_dim,
                                                       int32_t window, int64_t n_full,
                                                       int64_t n_local) {
  if (batch < 1 || seq_q < 0 || seq_kv < 1 || heads_q < 1 || heads_kv < 1 || head_dim != kD ||
      heads_q % heads_kv != 0 || window <= 0 || n_full < 0 || n_local < 0)
    return 0;
  const SplitPlan sp = split_plan(batch, seq_kv, heads_q, heads_kv, window, n_full, n_local);
  return sp.maxc > 1 ? sp.bytes : swattn_prefill_workspace_bytes(batch, seq_kv, heads_kv, head_dim);
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
  // Per-lane staging offsets inside a key tile are 32-bit: (rows of a tile) x
  // heads_kv x 256 bytes must stay below 2^31.
  if (heads_kv > 4096 || heads_q > 65536)
    return invalid("swattn_prefill_fwd: at most 4096 KV heads and 65536 query heads");
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
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return invalid("swattn_prefill_fwd: q, k, v and out must be 16-byte aligned");
  const size_t ws_need = swattn_prefill_workspace_bytes(batch, seq_kv, heads_kv, head_dim);
  if (workspace == nullptr || workspace_bytes < ws_need) {
    set_error("swattn_prefill_fwd: workspace smaller than swattn_prefill_workspace_bytes()");
    return SWATTN_EWORKSPACE;
  }
  if (!aligned256(workspace)) return invalid("swattn_prefill_fwd: workspace must be 256-byte aligned");

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
  p.total_q = static_cast<int32_t>(total_q);
  p.total_kv = static_cast<int32_t>(total_kv);
  p.kv_tiles = static_cast<int32_t>(kv_tiles_for(total_kv));
  p.hq = heads_q;
  p.hkv = heads_kv;
  p.group = group;
  p.window = window;
  p.c = scale_log2;
  // The key-range split runs when the plan asks for it and the workspace is
  // the larger size that swattn_prefill_split_workspace_bytes() returns.
  const SplitPlan sp = split_plan(batch, seq_kv, heads_q, heads_kv, window, n_full, n_local);
  const bool split = sp.maxc > 1 && workspace_bytes >= sp.bytes;
  p.maxc = split ? sp.maxc : 1;
  p.split_tiles = sp.tiles;
  char* ws = static_cast<char*>(workspace);
  p.part_o = split ? reinterpret_cast<float*>(ws + sp.off_o) : nullptr;
  p.part_lse = split ? reinterpret_cast<float*>(ws + sp.off_lse) : nullptr;
  p.part_n = split ? reinterpret_cast<int2*>(ws + sp.off_n) : nullptr;
  const int64_t grid = (static_cast<int64_t>(p.tiles[0]) * p.maxc + p.tiles[1]) * heads_kv;
  if (grid > INT32_MAX) return invalid("swattn_prefill_fwd: grid too large");
  const hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(vt_pack_kernel, dim3(p.kv_tiles, heads_kv), dim3(256), 0, st, p.v,
                     static_cast<uint16_t*>(workspace), p.total_kv, heads_kv, p.kv_tiles);
  const dim3 g3(static_cast<uint32_t>(grid)), b3(kThreads);
  if (split) {
    if (meta)
      hipLaunchKernelGGL((fwd_kernel<true, true>), g3, b3, 0, st, p);
    else
      hipLaunchKernelGGL((fwd_kernel<false, true>), g3, b3, 0, st, p);
  } else {
    if (meta)
      hipLaunchKernelGGL((fwd_kernel<true, false>), g3, b3, 0, st, p);
    else
      hipLaunchKernelGGL((fwd_kernel<false, false>), g3, b3, 0, st, p);
  }
  if (split && p.tiles[0] > 0)
    hipLaunchKernelGGL(fwd_merge_kernel,
                       dim3(static_cast<uint32_t>(static_cast<int64_t>(p.tiles[0]) * heads_kv *
                                                  kRowsPerItem * 32 / 256)),
                       dim3(256), 0, st, p);
  return launch_status("swattn_prefill_fwd");
}
