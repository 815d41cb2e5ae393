// Routed GQA prefill backward for gfx950 (MI355X): dQ, dK, dV of both Switch
// Attention branches from the forward's output and log2 LSE.
//
// Reference tags: V = swiattn_gqa_prefill_varlen.py, F = swiattn_gqa_prefill.py.
// The reference is forward-only (V:14-15); this is the derivative of its
// forward (V:103-249): per query row r (query head h of KV head h / G) and
// legal key j (V:134-137, V:186-196; F:145-155 without metadata),
//   P[r,j] = 2^(c * q_r.k_j - LSE_r)         (log2 LSE exported at V:236-241)
//   Delta_r = dO_r . O_r,   dS[r,j] = P[r,j] * (dO_r . v_j - Delta_r)
//   dq_r = s * sum_j dS[r,j] k_j,  dk_j = s * sum_r dS[r,j] q_r,
//   dv_j = sum_r P[r,j] dO_r        (s = sm_scale = c * ln 2)
// with dk_j / dv_j summed over the G query heads of the KV head.
//
// Design (MI355X-first):
// * Rows are ordered as in the forward (compacted query slot, head of the
//   group; head fastest), in blocks of 32.  bwd_prep_kernel computes Delta
//   once per row and writes, per (branch, KV head, block), a 1 KiB block of
//   row info: LSE, Delta, key bounds, the block's bounds summary, and each
//   row's element offset in Q / dO (-1 for a row that contributes nothing).
//   Q and dO themselves are never copied.
// * bwd_dkdv_kernel: one workgroup of eight waves (two per SIMD) per
//   (256-key tile, KV head); each wave keeps its 32 keys' K as MFMA B
//   operands in registers and dK^T, dV^T (128 d x 32 keys each) in
//   accumulators; the workgroup's V rows sit in LDS.  It streams the row
//   blocks that can see the tile (a contiguous block range per branch,
//   found by bwd_ranges_kernel with a wave-parallel search over the
//   monotone row bounds) through a three-slot LDS ring.  Each block's 32 Q and dO rows
//   are gathered from their positions by global_load_lds_dwordx4 (one
//   64-bit source address per lane), from the row offsets of the block's
//   info, which travels one block ahead through a four-slot info ring.
//   Four MFMA products per block: S = Q K^T, dP = dO V^T, dV^T += dO^T P,
//   dK^T += Q^T dS.  The A operands of the last two (Q^T, dO^T) come from
//   the same row-major blocks through transposing LDS reads
//   (ds_read_b64_tr_b16) that deliver the rows of each 16-row group in the
//   order the S / dP accumulators hold them, so those accumulators are the
//   B operands unchanged.
// * bwd_dq_kernel: one workgroup of eight waves per (branch, 256-row tile,
//   KV head), the forward's shape: each wave owns 32 rows, loads Q^T and
//   dO^T from the rows' positions as B operands, and streams K and V tiles
//   through a three-slot LDS ring.  Three products per 64-key tile: S^T =
//   K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T (K^T by transposing reads of
//   the K tile; dS^T as B operand straight from the accumulator).
// * Keys outside a row's range get S = -inf, so P = 0 exactly; a row with no
//   legal key (or a padding row) carries LSE = Delta = 0 and bounds [0, 0),
//   is masked everywhere and contributes nothing.
// * Grids of fewer than 512 (key tile, KV head) pairs split each pair over
//   its row blocks (up to 16 workgroups); bwd_dkdv_reduce_kernel sums the
//   fp32 partials in split order.  Pairs run longest first (the first key
//   tiles of each sequence are seen by the most rows).  When the longest
//   dQ row tile (the latest full rows see every earlier key) would set the
//   dQ kernel's length, row tiles longer than the estimated key tiles per
//   workgroup slot are cut into equal pieces of their key range; pieces
//   write fp32 partials that bwd_dq_reduce_kernel sums in piece order.
// * dQ is a separate pass (S and dP recomputed) rather than atomics from the
//   key-stationary pass, so every output is written once, deterministically.

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <algorithm>

#include "swattn_bwd_dkdv.inc"
#include "swattn_bwd_dq.inc"
#include "tiles.h"

namespace swattn {
namespace {

using namespace tiles;

constexpr int kThreads = 256;                          // prep / ranges workgroups
constexpr int kBwdWaves = 8;                           // dK/dV and dQ: two waves per SIMD
constexpr int kBwdThreads = kBwdWaves * 64;
constexpr int kBRows = 32;                             // rows per block
constexpr int kBlockBytes = kBRows * kRowBytes;        // 8 KiB row-major block in LDS
constexpr int kInfoBytes = 1024;                       // row info block
constexpr int kInfoLse = 0, kInfoDelta = 32, kInfoStart = 64, kInfoEnd = 96;   // word offsets
constexpr int kInfoMaxStart = 128, kInfoMinEnd = 129;
constexpr int kInfoRowOff = 96;                        // int64 offset: row element offsets (bytes 768..1023)
constexpr int kInfoRowOff32 = 160;                     // word offset: row byte offsets (bytes 640..767)
constexpr int kKeysDkv = kBwdWaves * 32;               // keys per dK/dV workgroup (32 per wave)
constexpr int kRowsPerItem = kBwdWaves * 32;           // rows per dQ workgroup (32 per wave)
constexpr int kVTileBytes = kKeysDkv * kRowBytes;      // the dK/dV workgroup's V rows: 64 KiB
// dK/dV LDS ring slot: Q block, dO block (row-major); three slots.  The
// blocks' info goes through its own four-slot ring, one block ahead.
constexpr int kStageBytes = 2 * kBlockBytes;
constexpr int kOffQ = 0, kOffDO = kBlockBytes;
constexpr int kRingSlots = 3;
constexpr int kInfoSlots = 4;
constexpr int kDkvLdsBytes = kVTileBytes + kRingSlots * kStageBytes + kInfoSlots * kInfoBytes;
// dK/dV split partials: per workgroup and wave, 32 float4 units per lane (16
// of dK^T, 16 of dV^T), unit-major so that a wave's store of one unit is
// 1 KiB contiguous.
constexpr int kPartUnits = 32;
constexpr size_t kPartBytesPerWg = static_cast<size_t>(kBwdWaves) * kPartUnits * 64 * 16;   // 256 KiB
// Below this many dK/dV workgroups (two rounds of one per CU on a 256-CU
// MI355X: the kernel's LDS allows one) the (key tile, KV head) pairs are
// split over their row blocks.
constexpr int64_t kDkvTargetWgs = 512;
constexpr int kDkvMaxSplit = 16;
// dQ workgroups that run at once (one per CU: the 96 KiB ring allows one).
constexpr int64_t kDqSlots = 256;
// dQ piece partials: per workgroup and wave, 16 float4 units per lane (dQ^T
// block d elements 4j .. 4j+3 in unit 4d + j), unit-major like the dK/dV ones.
constexpr int kDqPartUnits = 16;
constexpr size_t kDqPartBytesPerWg = static_cast<size_t>(kBwdWaves) * kDqPartUnits * 64 * 16;   // 128 KiB
constexpr int kDqMinTilesPerPiece = 4;   // 64-key tiles a dQ piece takes at least
// dQ LDS ring slot: K tile, V tile (16 KiB each); three slots.
constexpr int kQStageBytes = 2 * kTileBytes;

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  const int32_t* idx[2];     // [0] full list, [1] local list
  const int32_t* starts[2];  // metadata starts per branch (kMeta only)
  const int32_t* ends;       // metadata causal ends (kMeta only)
  int32_t count[2];          // slots per branch
  int32_t nrows[2];          // count * G
  int32_t blocks[2];         // ceil(nrows / 32)
  int32_t items[2];          // ceil(nrows / 128)
  int64_t blk_base[2];       // packed block of (branch b, head h, block i): blk_base[b] + h * blocks[b] + i
  char* info;                // [blocks][1 KiB]
  uint16_t* zero_row;        // 128 zeros: the gather source of rows that contribute nothing
  int32_t* ranges;           // [2][kv_tiles_dkv][2] block ranges
  float* dkv_part;           // dK/dV split partials (dkv_split > 1): [workgroup][8 waves][32][64 lanes] float4
  int32_t dkv_split;         // dK/dV workgroups per (key tile, KV head), over its row blocks
  int32_t dkv_batches;       // > 1: key tiles ordered tile-in-sequence-major over this many sequences
  float* dq_part;            // dQ piece partials (dq_chunk > 0): [workgroup][8 waves][16][64 lanes] float4
  int32_t* dq_nch;           // pieces per (row tile, KV head), written by piece 0 (dq_chunk > 0)
  int32_t dq_chunk;          // key tiles per dQ piece (0: row tiles are never cut)
  int32_t dq_maxc[2];        // workgroup slots per row tile of each branch
  int32_t seq_q, seq_kv, total_q, total_kv, kv_tiles_dkv;
  int32_t hq, hkv, group, window;
  float c;                   // sm_scale * log2(e)
  float scale;               // sm_scale
};

// A listed position outside [0, total_q) is never dereferenced: the host
// checks the lists before the launch, and this keeps a list changed after
// that check from turning into an out-of-bounds access.
__device__ __forceinline__ bool pos_ok(const BwdParams& p, int pos) {
  return static_cast<uint32_t>(pos) < static_cast<uint32_t>(p.total_q);
}

template <bool kMeta>
__device__ __forceinline__ void row_bounds(const BwdParams& p, int branch, int pos, int& ks,
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
  // An empty range keeps ks = ke.  F's rule with seq_q > seq_kv + window - 1
  // gives late local rows a start past their end (and past the next
  // sequence's first start); clipped, the starts are non-decreasing along
  // each list, as bwd_ranges_kernel's search needs.
  ks = min(ks, ke);
}

__device__ __forceinline__ int64_t packed_block(const BwdParams& p, int b, int kvh, int blk) {
  return p.blk_base[b] + static_cast<int64_t>(kvh) * p.blocks[b] + blk;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---------------------------------------------------------------------------
// Preparation: one workgroup per (branch, block of 32 rows, KV head).
// ---------------------------------------------------------------------------
template <bool kMeta>
__global__ __launch_bounds__(kThreads) void bwd_prep_kernel(const BwdParams p) {
  __shared__ int s_ks[kBRows], s_ke[kBRows];
  const int x = blockIdx.x, kvh = blockIdx.y;
  const int b = x < p.blocks[0] ? 0 : 1;
  const int blk = x - (b ? p.blocks[0] : 0);
  const int64_t pb = packed_block(p, b, kvh, blk);
  const int tid = threadIdx.x;
  const int rr = tid >> 3, part = tid & 7;   // row in block, 16 d values per thread
  const int r = blk * kBRows + rr;
  const int G = p.group;
  bool valid = r < p.nrows[b];
  int pos = 0, qh = 0, ks = 0, ke = 0;
  if (valid) {
    const int slot = r / G;
    qh = kvh * G + (r - slot * G);
    pos = p.idx[b][slot];
    valid = pos_ok(p, pos);   // otherwise a dead row: zeros, bounds [0, 0)
    if (valid)
      row_bounds<kMeta>(p, b, pos, ks, ke);
    else
      pos = 0;
  }
  const bool live = valid && ks < ke;
  const int64_t row_off = (static_cast<int64_t>(pos) * p.hq + qh) * kD;
  uint4 dv[2], ov[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) dv[i] = ov[i] = make_uint4(0, 0, 0, 0);
  if (live) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dv[i] = *reinterpret_cast<const uint4*>(p.dout + row_off + 16 * part + 8 * i);
      ov[i] = *reinterpret_cast<const uint4*>(p.o + row_off + 16 * part + 8 * i);
    }
  }
  float delta = 0.f;
  if (live) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t dw[4] = {dv[i].x, dv[i].y, dv[i].z, dv[i].w};
      const uint32_t ow[4] = {ov[i].x, ov[i].y, ov[i].z, ov[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        delta += bf16_lo(dw[e]) * bf16_lo(ow[e]) + bf16_hi(dw[e]) * bf16_hi(ow[e]);
    }
  }
  delta += __shfl_xor(delta, 1);
  delta += __shfl_xor(delta, 2);
  delta += __shfl_xor(delta, 4);

  // The gather source of every row that contributes nothing.
  if (x == 0 && kvh == 0 && tid < kRowBytes / 16)
    reinterpret_cast<uint4*>(p.zero_row)[tid] = make_uint4(0, 0, 0, 0);
  if (part == 0) {
    float* inf = reinterpret_cast<float*>(p.info + pb * kInfoBytes);
    int* infi = reinterpret_cast<int*>(inf);
    inf[kInfoLse + rr] = live ? p.lse[static_cast<int64_t>(pos) * p.hq + qh] : 0.f;
    inf[kInfoDelta + rr] = live ? delta : 0.f;
    infi[kInfoStart + rr] = live ? ks : 0;
    infi[kInfoEnd + rr] = live ? ke : 0;
    reinterpret_cast<int64_t*>(inf)[kInfoRowOff + rr] = live ? row_off : -1;
    // The same as a 32-bit byte offset for bwd_dkdv_wide_kernel's buffer
    // loads (only used where Q is below 2^31 bytes; past every range when
    // the row contributes nothing, so that its loads read zeros).
    reinterpret_cast<uint32_t*>(inf)[kInfoRowOff32 + rr] =
        live ? static_cast<uint32_t>(row_off * 2) : 0x80000000u;
    s_ks[rr] = live ? ks : INT_MAX;   // a dead row forces the mask on its block
    s_ke[rr] = live ? ke : INT_MIN;
  }
  __syncthreads();
  if (tid == 0) {
    int ms = INT_MIN, me = INT_MAX;
    for (int i = 0; i < kBRows; ++i) {
      ms = max(ms, s_ks[i]);
      me = min(me, s_ke[i]);
    }
    int* infi = reinterpret_cast<int*>(p.info + pb * kInfoBytes);
    infi[kInfoMaxStart] = ms;
    infi[kInfoMinEnd] = me;
  }
}

// ---------------------------------------------------------------------------
// Block ranges: for each branch and dK/dV key tile, the packed blocks whose
// rows can see a key of the tile.  Row bounds are non-decreasing along each
// list, so the slots that overlap [k0, k1) are [first with end > k0, first
// with start >= k1).
// ---------------------------------------------------------------------------
// The first slot in [lo, hi) of list b whose row bounds satisfy pred (false
// ... false, true ... true along the list), or hi.  A wave searches
// together: each step probes 64 evenly spaced slots at once and keeps the
// gap between the last false and the first true probe, so a list of n slots
// costs about log64(n) dependent loads instead of log2(n).  lo and hi stay
// wave-uniform (ballot), and every probe lies in [lo, hi).
template <bool kMeta, class Pred>
__device__ int wave_lower_bound(const BwdParams& p, int b, int lo, int hi, Pred pred) {
  const int lane = threadIdx.x & 63;
  while (lo < hi) {
    const int64_t span = hi - lo;
    const int probe = lo + static_cast<int>(span * lane / 64);
    const int pm = p.idx[b][probe];
    int ks, ke;
    row_bounds<kMeta>(p, b, pos_ok(p, pm) ? pm : 0, ks, ke);
    const uint64_t m = __builtin_amdgcn_ballot_w64(pred(ks, ke));
    if (m == 0) {
      lo += static_cast<int>(span * 63 / 64) + 1;   // past the last probe
    } else {
      const int first = __builtin_ctzll(m);
      hi = lo + static_cast<int>(span * first / 64);
      if (first > 0) lo += static_cast<int>(span * (first - 1) / 64) + 1;
    }
  }
  return lo;
}

// One wave per (branch, key tile).
template <bool kMeta>
__global__ __launch_bounds__(kThreads) void bwd_ranges_kernel(const BwdParams p) {
  const int i = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (i >= 2 * p.kv_tiles_dkv) return;   // whole waves
  const int b = i / p.kv_tiles_dkv, t = i - b * p.kv_tiles_dkv;
  const int k0 = t * kKeysDkv, k1 = min(k0 + kKeysDkv, p.total_kv);
  const int n = p.count[b];
  const int s_lo = wave_lower_bound<kMeta>(p, b, 0, n, [=](int, int ke) { return ke > k0; });
  const int s_hi = wave_lower_bound<kMeta>(p, b, s_lo, n, [=](int ks, int) { return ks >= k1; });
  int blo = 0, bhi = 0;
  if (s_lo < s_hi) {
    const int64_t G = p.group;
    blo = static_cast<int>((s_lo * G) / kBRows);
    bhi = static_cast<int>((s_hi * G + kBRows - 1) / kBRows);
  }
  if ((threadIdx.x & 63) == 0) {
    p.ranges[2 * i] = blo;
    p.ranges[2 * i + 1] = bhi;
  }
}

// ---------------------------------------------------------------------------
// dK / dV: one workgroup per (256-key tile, KV head), eight waves of 32 keys.
// ---------------------------------------------------------------------------
struct DkvPlan {
  int row[2];        // this lane's block row, per 1 KiB load
  uint32_t cb[2];    // byte offset inside that row of the chunk this lane fetches
  uint32_t voff[8];  // V rows: source offset from the tile's first key row, per 1 KiB load
};

// Waves 4p .. 4p+3 stage the four quarters of block part p (0 = Q, 1 = dO;
// row-major 256-byte rows, chunk swizzle swz): lane l of load i lands on
// byte 16 c of the part, c = 128 quarter + 64 i + l, i.e. on chunk position
// c % 16 of block row c / 16, and fetches the logical chunk that belongs
// there from that row's position in Q or dO.  The V tile (256 key rows,
// swizzle swz) is staged once: wave w loads rows 32w .. 32w+31, four rows
// per load.
__device__ __forceinline__ DkvPlan make_dkv_plan(const BwdParams& p, int kvh, int wave, int lane) {
  DkvPlan pl;
  const int quarter = wave & 3;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = 128 * quarter + 64 * i + lane;
    pl.row[i] = c >> 4;
    pl.cb[i] = static_cast<uint32_t>(((c & 15) ^ swz(c >> 4)) << 4);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 32 * wave + 4 * i + (lane >> 4);
    const int j = (lane & 15) ^ swz(row);
    pl.voff[i] = static_cast<uint32_t>(((row * p.hkv + kvh) * kD + 8 * j) * 2);
  }
  return pl;
}

// A block's Q and dO rows: two 1 KiB gathers per wave into the ring slot at
// LDS address slot, from the row offsets of the block's info (already in
// LDS at info).  A row with offset -1 is fetched from the zero row.
__device__ __forceinline__ void stage_rows(const BwdParams& p, const DkvPlan& pl, int wave,
                                           const char* info, uint32_t slot) {
  const int part = wave >> 2, quarter = wave & 3;
  const char* src = reinterpret_cast<const char*>(part == 0 ? p.q : p.dout);
  const int64_t* row_off = reinterpret_cast<const int64_t*>(info) + kInfoRowOff;
  const uint32_t dst = slot + part * kBlockBytes + quarter * (kBlockBytes / 4);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t ro = row_off[pl.row[i]];
    const char* a = (ro >= 0 ? src + 2 * ro : reinterpret_cast<const char*>(p.zero_row)) + pl.cb[i];
    dma16_gather(a, __builtin_amdgcn_readfirstlane(dst + 1024 * i));
  }
}

// A block's 1 KiB info into the info ring slot at LDS address slot (one
// load, issued by the last wave; the same load form as the row gathers, so
// that the loop's vmcnt counts cover one kind of load).
__device__ __forceinline__ void stage_info(const BwdParams& p, int lane, int64_t pb,
                                           uint32_t slot) {
  dma16_gather(p.info + pb * kInfoBytes + 16 * lane, __builtin_amdgcn_readfirstlane(slot));
}

typedef short i16x4 __attribute__((ext_vector_type(4)));

// A operand of X^T (32 d rows x 16 block rows, k-step s) read from the
// row-major block X in LDS with two transposing reads (ds_read_b64_tr_b16).
// In each 16-lane group, output lane i, element j of a read is element i%4
// of the 8 bytes that lane 4j + i/4 of the group addressed.  Lane 4j + q of
// group g = 2h + dh addresses row 16s + 8a + 4h + j, d = dbase + 16dh + 4q
// (read a = 0, 1), so output lane (m = 16dh + i, h) holds X[row][dbase + m]
// for the rows 16s + 8(t/4) + 4h + t%4, t = 0..7: the perm16 order in which
// the S / dP accumulators hold the same rows as B operands.  toff[s][a] is
// that address for dbase = 0; d block dblk adds 64 ((dblk ^ j) & 3), the
// high half of the row's chunk swizzle.
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
__device__ __forceinline__ bf16x8 read_xt(const char* xb, int off0, int off1) {
  __attribute__((address_space(3))) char* base = (__attribute__((address_space(3))) char*)(xb);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + off0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + off1));
  const i16x4 v[2] = {lo, hi};
  return __builtin_bit_cast(bf16x8, v);
}

// (key tile, KV head) of dK/dV pair rank r.  Pairs run in rank order, KV
// head fastest.  With dkv_batches > 1 (sequences of whole key tiles) tile i
// of every sequence comes before tile i+1 of any: the first tiles of a causal
// sequence are seen by the most rows, so the grid runs longest pairs first.
__device__ __forceinline__ void dkv_pair(const BwdParams& p, int r, int& t, int& kvh) {
  const int tr = r / p.hkv;
  kvh = r - tr * p.hkv;
  if (p.dkv_batches > 1) {
    const int per_seq = p.kv_tiles_dkv / p.dkv_batches;
    const int i = tr / p.dkv_batches;
    t = (tr - i * p.dkv_batches) * per_seq + i;
  } else {
    t = tr;
  }
}

// The bf16 dK / dV rows of one lane's key (lane half h) from its dK^T / dV^T
// accumulators: element e of block d is d-row 32d + 8(e/4) + 4h + e%4.
__device__ __forceinline__ void store_dkdv_rows(const BwdParams& p, int key, int kvh, int h,
                                                const f32x16 (&dkt)[4], const f32x16 (&dvt)[4]) {
  if (key >= p.total_kv) return;
  const int64_t base = (static_cast<int64_t>(key) * p.hkv + kvh) * kD + 4 * h;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 uk, uv;
      uk.x = pack_bf16x2(dkt[d][4 * j + 0] * p.scale, dkt[d][4 * j + 1] * p.scale);
      uk.y = pack_bf16x2(dkt[d][4 * j + 2] * p.scale, dkt[d][4 * j + 3] * p.scale);
      uv.x = pack_bf16x2(dvt[d][4 * j + 0], dvt[d][4 * j + 1]);
      uv.y = pack_bf16x2(dvt[d][4 * j + 2], dvt[d][4 * j + 3]);
      *reinterpret_cast<uint2*>(p.dk + base + 32 * d + 8 * j) = uk;
      *reinterpret_cast<uint2*>(p.dv + base + 32 * d + 8 * j) = uv;
    }
  }
}

// Float4 unit u of (workgroup wg, wave, lane) in the split partials: units
// 4d + j hold dK^T block d elements 4j .. 4j+3, units 16 + 4d + j the same of
// dV^T.
__device__ __forceinline__ float4* part_unit(const BwdParams& p, int64_t wg, int wave, int u,
                                             int lane) {
  return reinterpret_cast<float4*>(p.dkv_part) + ((wg * kBwdWaves + wave) * kPartUnits + u) * 64 +
         lane;
}

// Float4 unit u (= 4d + j: dQ^T block d elements 4j .. 4j+3) of (workgroup
// wg, wave, lane) in the dQ piece partials.
__device__ __forceinline__ float4* dq_part_unit(const BwdParams& p, int64_t wg, int wave, int u,
                                                int lane) {
  return reinterpret_cast<float4*>(p.dq_part) + ((wg * kBwdWaves + wave) * kDqPartUnits + u) * 64 +
         lane;
}

__global__ __attribute__((amdgpu_flat_work_group_size(kBwdThreads, kBwdThreads),
                          amdgpu_waves_per_eu(2, 2))) void bwd_dkdv_kernel(const BwdParams p) {
  // [V tile: 256 key rows][three Q / dO block slots][four info slots]
  __shared__ __attribute__((aligned(1024))) char smem[kDkvLdsBytes];
  const int tid = threadIdx.x;
  // The wave index as a scalar: per-wave choices (which block part a wave
  // stages, its source pointer) then stay scalar selects.
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, h = lane >> 5;
  // Workgroup = (pair rank, split s): the rank gives the (key tile t, KV
  // head) pair (dkv_pair); split s of dkv_split takes an equal share of the
  // pair's row blocks (all of them without a split).
  const int split = p.dkv_split;
  const int pair = blockIdx.x / split;
  const int s_idx = blockIdx.x - pair * split;
  int t, kvh;
  dkv_pair(p, pair, t, kvh);
  const int kw0 = t * kKeysDkv + 32 * wave;   // this wave's first key
  const int key = kw0 + n;                    // this lane's key (B column)

  // K of this lane's key as B operands: k-step kk holds d 16kk+8h .. +7.
  bf16x8 kf[8];
  if (key < p.total_kv) {
    const int64_t base = (static_cast<int64_t>(key) * p.hkv + kvh) * kD + 8 * h;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) kf[kk] = *reinterpret_cast<const bf16x8*>(p.k + base + 16 * kk);
  } else {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) kf[kk] = bf16x8{};
  }
  // Wait for the K loads with the builtin, before any LDS load is issued:
  // the compiler then knows they are complete.  Otherwise it keeps them
  // outstanding into the block loop and waits for them at their first use
  // there with vmcnt counts that also drain the next blocks' LDS loads.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  f32x16 dkt[4], dvt[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) dkt[d] = dvt[d] = f32x16{};

  const int nt = p.kv_tiles_dkv;
  const int b0lo = p.ranges[2 * t], b0hi = p.ranges[2 * t + 1];
  const int b1lo = p.ranges[2 * (nt + t)], b1hi = p.ranges[2 * (nt + t) + 1];
  const int n0 = max(b0hi - b0lo, 0), n1 = max(b1hi - b1lo, 0);
  const int chunk = (n0 + n1 + split - 1) / split;
  const int first = min(n0 + n1, s_idx * chunk);
  const int nb = min(n0 + n1 - first, chunk);   // this workgroup's blocks: first .. first+nb-1
  auto block_of = [&](int i) -> int64_t {
    const int a = first + i;
    return a < n0 ? packed_block(p, 0, kvh, b0lo + a) : packed_block(p, 1, kvh, b1lo + a - n0);
  };

  const DkvPlan pl = make_dkv_plan(p, kvh, wave, lane);
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t ring0 = lds0 + kVTileBytes;
  const uint32_t info0 = ring0 + kRingSlots * kStageBytes;
  const char* info_lds = smem + kVTileBytes + kRingSlots * kStageBytes;
  // The V tile, once: rows past total_kv fall outside the descriptor.
  if (nb > 0) {
    const int64_t row_bytes = static_cast<int64_t>(p.hkv) * kD * 2;
    const int64_t rest = (static_cast<int64_t>(p.total_kv) - static_cast<int64_t>(t) * kKeysDkv) * row_bytes;
    const i32x4 rv = make_rsrc(reinterpret_cast<const char*>(p.v) + static_cast<int64_t>(t) * kKeysDkv * row_bytes,
                               static_cast<uint32_t>(rest < 0xffffffffLL ? rest : 0xffffffffLL));
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dma16(rv, pl.voff[i], __builtin_amdgcn_readfirstlane(lds0 + (32 * wave + 4 * i) * kRowBytes));
  }
  // Operand offsets: Q / dO rows (A of S, dP): row n, chunk 2kk + h; V rows
  // (B of dP): key row 32 wave + n, chunk 2kk + h; Q^T / dO^T (A of dK^T,
  // dV^T): transposing reads, see read_xt.
  int aoff[8], toff[2];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) aoff[kk] = n * kRowBytes + (((2 * kk + h) ^ swz(n)) << 4);
  // Transposing reads for k-step 0 (k-step s adds 16 rows: 4096 bytes; the
  // swizzle's (row >> 2) & 3 does not change with it).
  const int tj = (lane >> 2) & 3, tq = lane & 3, tdh = (lane >> 4) & 1;
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int row = 8 * a + 4 * h + tj;
    const int clo = 2 * tdh + (tq >> 1);
    toff[a] = row * kRowBytes + ((clo ^ ((row >> 2) & 3)) << 4) + ((tq & 1) << 3);
  }
  const char* vrow = smem + 32 * wave * kRowBytes;

  // Three-slot row ring: block i+2's rows load while block i is computed;
  // the four-slot info ring runs one block further ahead (block i+3), so
  // that a block's row offsets are in LDS when its rows are gathered.  The
  // prologue stages the info of blocks 0..2 and, once it has landed, the
  // rows of blocks 0 and 1.  (The other waves' V loads may stay in flight:
  // block 0's wait covers them.)
  if (wave == kBwdWaves - 1) {
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (j < nb) stage_info(p, lane, block_of(j), info0 + j * kInfoBytes);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  asm volatile("s_barrier" ::: "memory");
  if (nb > 0) stage_rows(p, pl, wave, info_lds, ring0);
  if (nb > 1) stage_rows(p, pl, wave, info_lds + kInfoBytes, ring0 + kStageBytes);
  int slot = 0;
  for (int i = 0; i < nb; ++i) {
    // Block i's rows (and, before block 0, the V tile) are in LDS once every
    // wave's own loads up to them are complete.  Only block i+1's two row
    // gathers, the last loads a wave issued, may stay in flight; the info of
    // block i+2, issued before them, has landed.  Every wave has finished
    // block i-1, whose row slot and info slot the next loads overwrite.
    if (i + 1 < nb)
      asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (wave == kBwdWaves - 1 && i + 3 < nb)
      stage_info(p, lane, block_of(i + 3), info0 + ((i + 3) & 3) * kInfoBytes);
    if (i + 2 < nb) {
      const int s2slot = slot >= 1 ? slot - 1 : slot + 2;   // (i + 2) % 3
      stage_rows(p, pl, wave, info_lds + ((i + 2) & 3) * kInfoBytes,
                 ring0 + s2slot * kStageBytes);
    }
    const char* sb = smem + kVTileBytes + slot * kStageBytes;
    slot = slot == kRingSlots - 1 ? 0 : slot + 1;
    const float* inf = reinterpret_cast<const float*>(info_lds + (i & 3) * kInfoBytes);
    const int* infi = reinterpret_cast<const int*>(inf);

    f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const bf16x8 aq = *reinterpret_cast<const bf16x8*>(sb + kOffQ + aoff[kk]);
      const bf16x8 ad = *reinterpret_cast<const bf16x8*>(sb + kOffDO + aoff[kk]);
      const bf16x8 bv = *reinterpret_cast<const bf16x8*>(vrow + aoff[kk]);
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, kf[kk], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ad, bv, dp, 0, 0, 0);
    }
    // Element e of the accumulators is row 8(e/4) + 4h + e%4 of the block.
    const bool interior = infi[kInfoMaxStart] <= kw0 && infi[kInfoMinEnd] >= kw0 + 32;
    if (!interior) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int4 st = *reinterpret_cast<const int4*>(infi + kInfoStart + 8 * j + 4 * h);
        const int4 en = *reinterpret_cast<const int4*>(infi + kInfoEnd + 8 * j + 4 * h);
        if (key < st.x || key >= en.x) s[4 * j + 0] = -INFINITY;
        if (key < st.y || key >= en.y) s[4 * j + 1] = -INFINITY;
        if (key < st.z || key >= en.z) s[4 * j + 2] = -INFINITY;
        if (key < st.w || key >= en.w) s[4 * j + 3] = -INFINITY;
      }
    }
    bf16x8 pk[2], dsk[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 l4 = *reinterpret_cast<const float4*>(inf + kInfoLse + 8 * j + 4 * h);
      const float4 d4 = *reinterpret_cast<const float4*>(inf + kInfoDelta + 8 * j + 4 * h);
      const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
      const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[4 * j + e], p.c, -lv[e]));
        const float ds = pe * (dp[4 * j + e] - dv[e]);
        pk[j >> 1][4 * (j & 1) + e] = static_cast<__bf16>(pe);
        dsk[j >> 1][4 * (j & 1) + e] = static_cast<__bf16>(ds);
      }
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int dx = (((d ^ tj) & 3) << 6) + 16 * kRowBytes * s2;
        const bf16x8 ado = read_xt(sb + kOffDO, toff[0] + dx, toff[1] + dx);
        const bf16x8 aqt = read_xt(sb + kOffQ, toff[0] + dx, toff[1] + dx);
        dvt[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ado, pk[s2], dvt[d], 0, 0, 0);
        dkt[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aqt, dsk[s2], dkt[d], 0, 0, 0);
      }
    }
  }

  if (split == 1) {
    store_dkdv_rows(p, key, kvh, h, dkt, dvt);
  } else {
    // fp32 partials (zeros for a split with no blocks); bwd_dkdv_reduce_kernel
    // sums the splits in order and stores the rows.
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        *part_unit(p, blockIdx.x, wave, 4 * d + j, lane) =
            make_float4(dkt[d][4 * j], dkt[d][4 * j + 1], dkt[d][4 * j + 2], dkt[d][4 * j + 3]);
        *part_unit(p, blockIdx.x, wave, 16 + 4 * d + j, lane) =
            make_float4(dvt[d][4 * j], dvt[d][4 * j + 1], dvt[d][4 * j + 2], dvt[d][4 * j + 3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// bwd_dkdv_wide_kernel: bwd_dkdv_kernel's (key tile, KV head) pairs with four
// waves of 64 keys, one wave per SIMD, for grids that need no split.  Each
// LDS read of a block's Q or dO operand then feeds two MFMAs (both 32-key
// halves of the wave), and the per-lane state (dK^T and dV^T in AGPRs; K,
// the score and dP tiles and their bf16 packs in VGPRs) exceeds what a
// compiler-allocated kernel gets, so the block loop is the generated
// assembly of gen_bwd_dkdv.py.  This C++ part resolves the pair, its row
// blocks and the per-lane offsets, and hands them to the loop through LDS.
// ---------------------------------------------------------------------------
constexpr int kDkvWideLdsBytes = SWATTN_BWD_DKDV_LDS_BYTES;
constexpr int kDkvAuxGroups = SWATTN_BWD_DKDV_AUX_GROUPS;
static_assert(SWATTN_BWD_DKDV_RING_OFF == kVTileBytes, "the V tile precedes the row ring");
static_assert(4 * kDkvAuxGroups * 1024 <= 2 * 2 * kBlockBytes, "the inputs fit in ring slots 2-3");

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bwd_dkdv_wide_kernel(const BwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kDkvWideLdsBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, hh = lane >> 5;
  // Workgroup = (pair rank, split s), as in bwd_dkdv_kernel: split s of
  // dkv_split takes an equal share of the pair's row blocks in the loop's
  // order (all of them without a split) and leaves fp32 partials.
  const int split = p.dkv_split;
  const int pair = blockIdx.x / split;
  const int s_idx = blockIdx.x - pair * split;
  int t, kvh;
  dkv_pair(p, pair, t, kvh);
  const int nt = p.kv_tiles_dkv;
  const int b0lo = p.ranges[2 * t], b0hi = p.ranges[2 * t + 1];
  const int b1lo = p.ranges[2 * (nt + t)], b1hi = p.ranges[2 * (nt + t) + 1];
  const int n0 = max(b0hi - b0lo, 0), n1 = max(b1hi - b1lo, 0);
  const int chunk = (n0 + n1 + split - 1) / split;
  const int first = min(n0 + n1, s_idx * chunk);
  const int nb = min(n0 + n1 - first, chunk);
  const int pb0 = static_cast<int>(packed_block(p, 0, kvh, b0lo));
  const int pb1 = static_cast<int>(packed_block(p, 1, kvh, b1lo)) - n0;
  const int kw0 = t * kKeysDkv + 64 * wave;
  const uint32_t krowbytes = static_cast<uint32_t>(p.hkv) * kRowBytes;
  const uint32_t lds0 = lds_addr(smem);
  constexpr uint32_t kOff = 0x80000000u;   // beyond every descriptor's range: dropped

  // Per-lane inputs of the loop (group g at aux + 1024 g + 16 lane).
  uint32_t w[kDkvAuxGroups * 4];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    const int key = kw0 + 32 * kh + j;
    const bool in = key < p.total_kv;
    const uint32_t row = static_cast<uint32_t>(key) * static_cast<uint32_t>(p.hkv) + kvh;
    w[kh] = in ? row * kRowBytes + 16 * hh : kOff;
    w[2 + kh] = in ? row * kRowBytes + 8 * hh : kOff;
  }
  w[4] = lds0 + kVTileBytes + j * kRowBytes + ((hh ^ swz(j)) << 4);
  w[5] = lds0 + (64 * wave + j) * kRowBytes + ((hh ^ swz(j)) << 4);
#pragma unroll
  for (int L = 0; L < 2; ++L)
    w[6 + L] = 16 * ((lane & 15) ^ ((((lane >> 4) & 3) << 2) | ((2 * wave + L) & 3)));
  const int tj = (lane >> 2) & 3, tq = lane & 3, tdh = (lane >> 4) & 1;
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int row = 8 * a + 4 * hh + tj;
    const int clo = 2 * tdh + (tq >> 1);
    const uint32_t toff = lds0 + kVTileBytes + row * kRowBytes + ((clo ^ ((row >> 2) & 3)) << 4) + ((tq & 1) << 3);
#pragma unroll
    for (int db = 0; db < 4; ++db) w[8 + 2 * db + a] = toff + (((db ^ tj) & 3) << 6);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    w[16 + q] = (64 * wave + (lane >> 4)) * krowbytes +
                16 * ((lane & 15) ^ ((((lane >> 4) & 3) << 2) | q));
  w[20] = kw0 + j;
  w[21] = 16 * hh;
  w[22] = 4 * kInfoRowOff32 + 32 * wave + 4 * (lane >> 4);
  w[23] = 0;
  const uint32_t aux = lds0 + SWATTN_BWD_DKDV_AUX_OFF + wave * kDkvAuxGroups * 1024;
  {
    uint4* a = reinterpret_cast<uint4*>(smem + (aux - lds0) + 16 * lane);
#pragma unroll
    for (int g = 0; g < kDkvAuxGroups; ++g)
      a[64 * g] = make_uint4(w[4 * g], w[4 * g + 1], w[4 * g + 2], w[4 * g + 3]);
  }

  const uint32_t qbytes = static_cast<uint32_t>(p.total_q) * static_cast<uint32_t>(p.hq) * kRowBytes;
  const uint32_t kvbytes = static_cast<uint32_t>(p.total_kv) * krowbytes;
  const i32x4 qrsrc = make_rsrc(p.q, qbytes);
  const i32x4 dorsrc = make_rsrc(p.dout, qbytes);
  const uint32_t nblocks = static_cast<uint32_t>(p.blk_base[1] + static_cast<int64_t>(p.hkv) * p.blocks[1]);
  const i32x4 irsrc = make_rsrc(p.info, nblocks * kInfoBytes);
  const i32x4 krsrc = make_rsrc(p.k, kvbytes);
  const i32x4 dkrsrc = make_rsrc(p.dk, kvbytes);
  const i32x4 dvrsrc = make_rsrc(p.dv, kvbytes);
  // The V tile: from its first key row (head kvh) to the end of V.
  const uint64_t vbase = reinterpret_cast<uint64_t>(p.v) +
                         (static_cast<uint64_t>(t) * kKeysDkv * p.hkv + kvh) * kRowBytes;
  const int vbytes = static_cast<int>(static_cast<int64_t>(kvbytes) -
                                      static_cast<int64_t>(t) * kKeysDkv * krowbytes -
                                      static_cast<int64_t>(kvh) * kRowBytes);
  const uint32_t vb_lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(vbase));
  const uint32_t vb_hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(vbase >> 32));
  const uint64_t vb64 = (static_cast<uint64_t>(vb_hi) << 32) | vb_lo;
  const float c = p.c, scale = p.scale;
  // This wave's split partials: the reduce's waves 2 wave and 2 wave + 1.
  const char* part = split > 1 ? reinterpret_cast<const char*>(p.dkv_part) +
                                     (static_cast<int64_t>(blockIdx.x) * kBwdWaves + 2 * wave) * kPartUnits * 1024
                               : reinterpret_cast<const char*>(p.dk);
  const i32x4 prsrc = make_rsrc(part, split > 1 ? 2 * kPartUnits * 1024 : 0);
  asm volatile(SWATTN_BWD_DKDV_ASM
               :
               : [qrsrc] "s"(qrsrc), [dorsrc] "s"(dorsrc), [irsrc] "s"(irsrc), [krsrc] "s"(krsrc),
                 [dkrsrc] "s"(dkrsrc), [dvrsrc] "s"(dvrsrc), [vbase] "s"(vb64),
                 [vbytes] "s"(__builtin_amdgcn_readfirstlane(vbytes)),
                 [nblk] "s"(__builtin_amdgcn_readfirstlane(nb)),
                 [pb1n] "s"(__builtin_amdgcn_readfirstlane(pb1 + n0)),
                 [pbf] "s"(__builtin_amdgcn_readfirstlane(pb0 + n0 - 1 - first)),
                 [pb1] "s"(__builtin_amdgcn_readfirstlane(pb1 + first)),
                 [prsrc] "s"(prsrc), [split] "s"(__builtin_amdgcn_readfirstlane(split > 1 ? 1 : 0)),
                 [kw0] "s"(__builtin_amdgcn_readfirstlane(kw0)),
                 [krow4] "s"(__builtin_amdgcn_readfirstlane(static_cast<int>(4 * krowbytes))),
                 [vl] "s"(__builtin_amdgcn_readfirstlane(lds0 + 64 * wave * kRowBytes)),
                 [wl] "s"(__builtin_amdgcn_readfirstlane(lds0 + 2048 * wave)),
                 [info0] "s"(__builtin_amdgcn_readfirstlane(lds0 + SWATTN_BWD_DKDV_INFO_OFF)),
                 [aux] "s"(__builtin_amdgcn_readfirstlane(aux)), [c] "s"(c), [scale] "s"(scale)
               : SWATTN_BWD_DKDV_CLOBBERS);
}

// dK / dV of split pairs: one thread per (pair, wave, float4 unit, lane).
// It sums that unit over the splits in split order (deterministic) and stores
// its four bf16 values where the unsplit kernel's epilogue would.
static_assert(kPartUnits == 32 && kBwdWaves == 8, "the reduce's thread index splits 6 + 5 + 3 bits");
__global__ __launch_bounds__(kThreads) void bwd_dkdv_reduce_kernel(const BwdParams p) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int lane = static_cast<int>(id & 63);
  const int u = static_cast<int>((id >> 6) & (kPartUnits - 1));
  const int wave = static_cast<int>((id >> 11) & (kBwdWaves - 1));
  const int pair = static_cast<int>(id >> 14);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp = 0; sp < p.dkv_split; ++sp) {
    const float4 a = *part_unit(p, static_cast<int64_t>(pair) * p.dkv_split + sp, wave, u, lane);
    acc.x += a.x;
    acc.y += a.y;
    acc.z += a.z;
    acc.w += a.w;
  }
  int t, kvh;
  dkv_pair(p, pair, t, kvh);
  const int key = t * kKeysDkv + 32 * wave + (lane & 31);
  if (key >= p.total_kv) return;
  // Unit 4d + j (+16 for dV): elements 4j .. 4j+3 of block d, i.e. d-rows
  // 32d + 8j + 4h .. +3 of the key (lane half h).
  const bool is_v = u >= 16;
  const int d = (u & 15) >> 2, j = u & 3;
  const float sc = is_v ? 1.0f : p.scale;
  uint2 w;
  w.x = pack_bf16x2(acc.x * sc, acc.y * sc);
  w.y = pack_bf16x2(acc.z * sc, acc.w * sc);
  uint16_t* dst = is_v ? p.dv : p.dk;
  *reinterpret_cast<uint2*>(dst + (static_cast<int64_t>(key) * p.hkv + kvh) * kD + 4 * (lane >> 5) +
                            32 * d + 8 * j) = w;
}

// ---------------------------------------------------------------------------
// dQ: one workgroup per (branch, 256-row tile, KV head), eight waves of 32 rows.
// ---------------------------------------------------------------------------
constexpr int kDqLoads = kBN / kBwdWaves / 4;   // 1 KiB loads per wave per K (or V) tile
struct DqPlan {
  uint32_t koff[kDqLoads];   // K / V row chunk offsets from the tile's first key row
  uint32_t lds_w;            // this wave's byte offset inside a 16 KiB tile
};

// Wave w stages key rows 8w .. 8w+7 of K and V, 1 KiB (4 key rows) per load;
// lane l lands on 16-byte position l of the load and fetches the logical
// chunk that belongs there (chunk swizzle swz).
__device__ __forceinline__ DqPlan make_dq_plan(const BwdParams& p, int kvh, int wave, int lane) {
  DqPlan pl;
#pragma unroll
  for (int i = 0; i < kDqLoads; ++i) {
    const int row = 4 * kDqLoads * wave + 4 * i + (lane >> 4);
    const int j = (lane & 15) ^ swz(row);
    pl.koff[i] = static_cast<uint32_t>(((row * p.hkv + kvh) * kD + 8 * j) * 2);
  }
  pl.lds_w = 4 * kDqLoads * wave * kRowBytes;
  return pl;
}

__device__ __forceinline__ void stage_dq(const BwdParams& p, const DqPlan& pl, int kvh, int tk,
                                         uint32_t slot) {
  const int64_t row_bytes = static_cast<int64_t>(p.hkv) * kD * 2;
  const int64_t rest = (static_cast<int64_t>(p.total_kv) - static_cast<int64_t>(tk) * kBN) * row_bytes;
  const uint32_t nrec = static_cast<uint32_t>(rest < 0xffffffffLL ? rest : 0xffffffffLL);
  const int64_t kv_off = static_cast<int64_t>(tk) * kBN * row_bytes;
  const i32x4 rk = make_rsrc(reinterpret_cast<const char*>(p.k) + kv_off, nrec);
  const i32x4 rv = make_rsrc(reinterpret_cast<const char*>(p.v) + kv_off, nrec);
#pragma unroll
  for (int i = 0; i < kDqLoads; ++i) {
    const uint32_t o = slot + pl.lds_w + 4 * i * kRowBytes;
    dma16(rk, pl.koff[i], __builtin_amdgcn_readfirstlane(o));
    dma16(rv, pl.koff[i], __builtin_amdgcn_readfirstlane(o + kTileBytes));
  }
}

__global__ __attribute__((amdgpu_flat_work_group_size(kBwdThreads, kBwdThreads),
                          amdgpu_waves_per_eu(2, 2))) void bwd_dq_kernel(const BwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kRingSlots * kQStageBytes];
  __shared__ int s_range[2 * kBwdWaves];
  const int tid = threadIdx.x;
  // The wave index as a scalar: per-wave choices (which block part a wave
  // stages, its source pointer) then stay scalar selects.
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, h = lane >> 5;
  // Workgroup = ((row tile t, piece slot s), KV head), KV head fastest; a
  // row tile of branch b has dq_maxc[b] consecutive slots.
  const int kvh = blockIdx.x % p.hkv;
  const int ts = blockIdx.x / p.hkv;
  const int full_slots = p.items[0] * p.dq_maxc[0];
  const int t = ts < full_slots ? ts / p.dq_maxc[0]
                                : p.items[0] + (ts - full_slots) / p.dq_maxc[1];
  const int s_idx = ts < full_slots ? ts - t * p.dq_maxc[0]
                                    : ts - full_slots - (t - p.items[0]) * p.dq_maxc[1];
  const int b = t < p.items[0] ? 0 : 1;
  // Latest positions first in each branch (longest rows first).
  const int item = b == 0 ? p.items[0] - 1 - t : p.items[0] + p.items[1] - 1 - t;
  const int blk = item * (kRowsPerItem / kBRows) + wave;
  const bool blk_ok = blk < p.blocks[b];
  const int64_t pb = packed_block(p, b, kvh, blk_ok ? blk : 0);
  const int r = blk * kBRows + n;
  const bool valid = blk_ok && r < p.nrows[b];

  // The row's element offset in Q / dO (-1: the row contributes nothing, its
  // operands are zeros and its bounds empty).
  float lse = 0.f, delta = 0.f;
  int ks = 0, ke = 0;
  int64_t row_off = -1;
  bf16x8 qf[8], dof[8];
  if (valid) {
    const float* inf = reinterpret_cast<const float*>(p.info + pb * kInfoBytes);
    const int* infi = reinterpret_cast<const int*>(inf);
    lse = inf[kInfoLse + n];
    delta = inf[kInfoDelta + n];
    ks = infi[kInfoStart + n];
    ke = infi[kInfoEnd + n];
    row_off = reinterpret_cast<const int64_t*>(inf)[kInfoRowOff + n];
  }
  const bool has = valid && ks < ke;
  const int w_min_s = wave_min(has ? ks : INT_MAX);
  const int w_max_e = wave_max(has ? ke : INT_MIN);
  if (lane == 0) {
    s_range[wave] = w_min_s;
    s_range[kBwdWaves + wave] = w_max_e;
  }
  __syncthreads();
  int g_s = INT_MAX, g_e = INT_MIN;
#pragma unroll
  for (int i = 0; i < kBwdWaves; ++i) {
    g_s = min(g_s, s_range[i]);
    g_e = max(g_e, s_range[kBwdWaves + i]);
  }
  const int t_all0 = g_e > g_s ? g_s / kBN : 0;
  const int t_all1 = g_e > g_s ? (g_e + kBN - 1) / kBN : 0;
  // This piece's key tiles [t_begin, t_end): a row tile longer than dq_chunk
  // tiles is cut into nch (at most dq_maxc[b]) equal pieces; slots past nch
  // have nothing to do (uniform over the workgroup: every thread computed
  // the same range).
  int t_begin = t_all0, t_end = t_all1;
  bool piece = false;
  if (p.dq_chunk > 0) {
    const int len = t_all1 - t_all0;
    const int nch = max(1, min(p.dq_maxc[b], (len + p.dq_chunk - 1) / p.dq_chunk));
    if (s_idx >= nch) return;
    if (s_idx == 0 && tid == 0) p.dq_nch[t * p.hkv + kvh] = nch;
    piece = nch > 1;
    const int plen = (len + nch - 1) / nch;
    t_begin = t_all0 + min(len, s_idx * plen);
    t_end = min(t_all1, t_begin + plen);
  }
  // Q and dO rows (after the exchange, so that unused piece slots load
  // nothing).  As in the dK/dV kernel: the row loads complete here, known to
  // the compiler, so that no wait in the tile loop drains the tile LDS loads.
  if (row_off >= 0) {
    const uint16_t* qrow = p.q + row_off + 8 * h;
    const uint16_t* drow = p.dout + row_off + 8 * h;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      qf[kk] = *reinterpret_cast<const bf16x8*>(qrow + 16 * kk);
      dof[kk] = *reinterpret_cast<const bf16x8*>(drow + 16 * kk);
    }
  } else {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = dof[kk] = bf16x8{};
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  // Tiles inside the range of every row this wave stores need no mask.  A
  // stored row with no key (start = end = 0) must see every tile masked, so
  // it counts as start = +inf, end = -inf; lanes that store nothing do not
  // count (their columns of the products are independent and discarded).
  const int w_max_s = __builtin_amdgcn_readfirstlane(
      wave_max(valid ? (has ? ks : INT_MAX) : INT_MIN));
  const int w_min_e = __builtin_amdgcn_readfirstlane(
      wave_min(valid ? (has ? ke : INT_MIN) : INT_MAX));
  const int it0 = w_max_s > INT_MAX - kBN ? INT_MAX : (w_max_s + kBN - 1) / kBN;
  const int it1 = w_min_e <= 0 ? 0 : w_min_e / kBN;

  // K / V rows (A of S^T, dP^T): key row n (+32), chunk 2kk + h.  K^T (A of
  // dQ^T): transposing reads of the K tile, as read_xt describes (rows are
  // keys; k-step s2 adds 16 key rows).
  int koff[8], toff[2];
  {
    const int kx = h ^ swz(n);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) koff[kk] = n * kRowBytes + (((2 * kk) ^ kx) << 4);
  }
  const int tj = (lane >> 2) & 3, tq = lane & 3, tdh = (lane >> 4) & 1;
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int row = 8 * a + 4 * h + tj;
    const int clo = 2 * tdh + (tq >> 1);
    toff[a] = row * kRowBytes + ((clo ^ ((row >> 2) & 3)) << 4) + ((tq & 1) << 3);
  }
  const DqPlan pl = make_dq_plan(p, kvh, wave, lane);
  const uint32_t lds0 = lds_addr(smem);
  f32x16 dqt[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) dqt[d] = f32x16{};

  // Three-slot ring: tile j+2 loads while tile j is computed.
  if (t_end > t_begin) stage_dq(p, pl, kvh, t_begin, lds0);
  if (t_end > t_begin + 1) stage_dq(p, pl, kvh, t_begin + 1, lds0 + kQStageBytes);
  int slot = 0;
  for (int j = t_begin; j < t_end; ++j) {
    // Tile j is in LDS once every wave's loads up to it are complete (tile
    // j+1's 2 kDqLoads loads may stay in flight); every wave has finished
    // tile j-1, whose slot the next loads overwrite.
    static_assert(kDqLoads == 2, "the wait below allows four loads in flight");
    if (j + 1 < t_end)
      asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (j + 2 < t_end) {
      const int s2slot = slot >= 1 ? slot - 1 : slot + 2;   // (j - t_begin + 2) % 3
      stage_dq(p, pl, kvh, j + 2, lds0 + s2slot * kQStageBytes);
    }
    const char* sk = smem + slot * kQStageBytes;
    slot = slot == kRingSlots - 1 ? 0 : slot + 1;
    const int key0 = j * kBN;
    if (!(key0 < w_max_e && key0 + kBN > w_min_s)) continue;
    const char* sv = sk + kTileBytes;
    f32x16 s0 = f32x16{}, s1 = f32x16{}, p0 = f32x16{}, p1 = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(sk + koff[kk]);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(sk + koff[kk] + 32 * kRowBytes);
      const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(sv + koff[kk]);
      const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(sv + koff[kk] + 32 * kRowBytes);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[kk], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[kk], s1, 0, 0, 0);
      p0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b0, dof[kk], p0, 0, 0, 0);
      p1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b1, dof[kk], p1, 0, 0, 0);
    }
    // Element 4j+i of block kb is key key0 + 32kb + 8j + 4h + i of this row.
    if (j < it0 || j >= it1) {
      const int lo = ks - key0 - 4 * h, hi = ke - key0 - 4 * h;
      const uint32_t span = hi > lo ? static_cast<uint32_t>(hi - lo) : 0u;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 8 * jj + i;
          if (static_cast<uint32_t>(e - lo) >= span) s0[4 * jj + i] = -INFINITY;
          if (static_cast<uint32_t>(e + 32 - lo) >= span) s1[4 * jj + i] = -INFINITY;
        }
      }
    }
    bf16x8 dsk[4];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pa = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[e], p.c, -lse));
      const float pc = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[e], p.c, -lse));
      dsk[e >> 3][e & 7] = static_cast<__bf16>(pa * (p0[e] - delta));
      dsk[2 + (e >> 3)][e & 7] = static_cast<__bf16>(pc * (p1[e] - delta));
    }
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int dx = (((d ^ tj) & 3) << 6) + 16 * kRowBytes * s2;
        const bf16x8 at = read_xt(sk, toff[0] + dx, toff[1] + dx);
        dqt[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(at, dsk[s2], dqt[d], 0, 0, 0);
      }
    }
  }

  const int G = p.group;
  if (piece) {
    // fp32 partials (zeros for a piece with no tiles); bwd_dq_reduce_kernel
    // sums the pieces in order and stores the rows.
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *dq_part_unit(p, blockIdx.x, wave, 4 * d + j, lane) =
            make_float4(dqt[d][4 * j], dqt[d][4 * j + 1], dqt[d][4 * j + 2], dqt[d][4 * j + 3]);
    }
    return;
  }
  const int q_slot = r / G;
  const int pos = valid ? p.idx[b][q_slot] : 0;
  if (valid && pos_ok(p, pos)) {
    const int qh = kvh * G + (r - q_slot * G);
    uint16_t* row = p.dq + (static_cast<int64_t>(pos) * p.hq + qh) * kD + 4 * h;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint2 u;
        u.x = pack_bf16x2(dqt[d][4 * j + 0] * p.scale, dqt[d][4 * j + 1] * p.scale);
        u.y = pack_bf16x2(dqt[d][4 * j + 2] * p.scale, dqt[d][4 * j + 3] * p.scale);
        *reinterpret_cast<uint2*>(row + 32 * d + 8 * j) = u;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// bwd_dq_wide_kernel: bwd_dq_kernel's work items with four waves of 64 rows,
// one wave per SIMD.  Each K / V operand read from LDS then feeds two MFMAs
// (both 32-row blocks of the wave), and the per-lane state (dQ^T, Q^T and
// dO^T in AGPRs; two score tiles, the dP tile and the operand staging in
// VGPRs) exceeds what a compiler-allocated kernel gets, so the tile loop is
// the generated assembly of gen_bwd_dq.py.  This C++ part resolves the
// rows, the tile range and pieces exactly as bwd_dq_kernel does and hands
// the loop its per-lane inputs through LDS (the loop needs every VGPR).
// ---------------------------------------------------------------------------
constexpr int kDqWideLdsBytes = SWATTN_BWD_DQ_LDS_BYTES;
static_assert(kDqWideLdsBytes == 8 * kTileBytes, "four-slot K and V rings of the generated loop");
constexpr int kDqAuxGroups = SWATTN_BWD_DQ_AUX_GROUPS;
static_assert(4 * SWATTN_BWD_DQ_EPI_REGION <= 3 * kTileBytes, "the dq staging fits in K slots 0-2");
// Per-lane inputs: group g of wave w at aux(w) + 1024 g + 16 lane, with
// aux(w) in K slot 3 (waves 0-1) or V slot 3 (waves 2-3).
__device__ __forceinline__ int dq_aux_offset(int wave) {
  return wave < 2 ? 3 * kTileBytes + wave * kDqAuxGroups * 1024
                  : 7 * kTileBytes + (wave - 2) * kDqAuxGroups * 1024;
}
static_assert(2 * kDqAuxGroups * 1024 <= kTileBytes, "two waves' inputs fit in a ring slot");

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bwd_dq_wide_kernel(const BwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kDqWideLdsBytes];
  __shared__ int s_range[8];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, h = lane >> 5;
  // Workgroup = ((row tile t, piece slot s), KV head) as in bwd_dq_kernel.
  const int kvh = blockIdx.x % p.hkv;
  const int ts = blockIdx.x / p.hkv;
  const int full_slots = p.items[0] * p.dq_maxc[0];
  const int t = ts < full_slots ? ts / p.dq_maxc[0]
                                : p.items[0] + (ts - full_slots) / p.dq_maxc[1];
  const int s_idx = ts < full_slots ? ts - t * p.dq_maxc[0]
                                    : ts - full_slots - (t - p.items[0]) * p.dq_maxc[1];
  const int b = t < p.items[0] ? 0 : 1;
  const int item = b == 0 ? p.items[0] - 1 - t : p.items[0] + p.items[1] - 1 - t;

  // This lane's two rows: row blocks 2 wave and 2 wave + 1 of the item.
  float lse[2], delta[2];
  int ks[2], ke[2], r[2];
  int64_t row_off[2];
  bool valid[2], has[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int blk = item * (kRowsPerItem / kBRows) + 2 * wave + rb;
    const bool blk_ok = blk < p.blocks[b];
    r[rb] = blk * kBRows + n;
    valid[rb] = blk_ok && r[rb] < p.nrows[b];
    lse[rb] = delta[rb] = 0.f;
    ks[rb] = ke[rb] = 0;
    row_off[rb] = -1;
    if (valid[rb]) {
      const float* inf = reinterpret_cast<const float*>(p.info + packed_block(p, b, kvh, blk) * kInfoBytes);
      const int* infi = reinterpret_cast<const int*>(inf);
      lse[rb] = inf[kInfoLse + n];
      delta[rb] = inf[kInfoDelta + n];
      ks[rb] = infi[kInfoStart + n];
      ke[rb] = infi[kInfoEnd + n];
      row_off[rb] = reinterpret_cast<const int64_t*>(inf)[kInfoRowOff + n];
    }
    has[rb] = valid[rb] && ks[rb] < ke[rb];
  }
  const int w_min_s = wave_min(min(has[0] ? ks[0] : INT_MAX, has[1] ? ks[1] : INT_MAX));
  const int w_max_e = wave_max(max(has[0] ? ke[0] : INT_MIN, has[1] ? ke[1] : INT_MIN));
  if (lane == 0) {
    s_range[wave] = w_min_s;
    s_range[4 + wave] = w_max_e;
  }
  __syncthreads();
  int g_s = INT_MAX, g_e = INT_MIN;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    g_s = min(g_s, s_range[i]);
    g_e = max(g_e, s_range[4 + i]);
  }
  const int t_all0 = g_e > g_s ? g_s / kBN : 0;
  const int t_all1 = g_e > g_s ? (g_e + kBN - 1) / kBN : 0;
  int t_begin = t_all0, t_end = t_all1;
  bool piece = false;
  if (p.dq_chunk > 0) {
    const int len = t_all1 - t_all0;
    const int nch = max(1, min(p.dq_maxc[b], (len + p.dq_chunk - 1) / p.dq_chunk));
    if (s_idx >= nch) return;
    if (s_idx == 0 && tid == 0) p.dq_nch[t * p.hkv + kvh] = nch;
    piece = nch > 1;
    const int plen = (len + nch - 1) / nch;
    t_begin = t_all0 + min(len, s_idx * plen);
    t_end = min(t_all1, t_begin + plen);
  }
  const int n_tiles = max(t_end - t_begin, 0);
  // Tiles inside the range of every row this wave stores need no mask (a
  // stored row with no key counts as start = +inf, end = -inf; lanes that
  // store nothing do not count).
  int ms = INT_MIN, me = INT_MAX;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    if (valid[rb]) {
      ms = max(ms, has[rb] ? ks[rb] : INT_MAX);
      me = min(me, has[rb] ? ke[rb] : INT_MIN);
    }
  }
  const int w_max_s = __builtin_amdgcn_readfirstlane(wave_max(ms));
  const int w_min_e = __builtin_amdgcn_readfirstlane(wave_min(me));
  const int it0 = (w_max_s > INT_MAX - kBN ? INT_MAX / 2 : (w_max_s + kBN - 1) / kBN) - t_begin;
  const int it1 = (w_min_e <= 0 ? 0 : w_min_e / kBN) - t_begin;

  // Per-lane inputs of the loop, into LDS (read back by the same lane).
  constexpr uint32_t kOff = 0x80000000u;   // beyond every descriptor's range: dropped
  const uint32_t lds0 = lds_addr(smem);
  uint32_t w[kDqAuxGroups * 4];
  const int G = p.group;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    // dq row: every valid row is written (zeros for a row with no key)
    const int q_slot = r[rb] / G;
    const int pos = valid[rb] ? p.idx[b][q_slot] : 0;
    const bool store = valid[rb] && pos_ok(p, pos);
    const int qh = kvh * G + (r[rb] - q_slot * G);
    w[0 + rb] = store ? static_cast<uint32_t>(((static_cast<int64_t>(pos) * p.hq + qh) * kD + 4 * h) * 2)
                      : kOff;
    w[2 + rb] = row_off[rb] >= 0 ? static_cast<uint32_t>(row_off[rb] * 2 + 16 * h) : kOff;
    w[4 + rb] = __float_as_uint(-lse[rb]);
    w[6 + rb] = __float_as_uint(delta[rb]);
    w[8 + rb] = static_cast<uint32_t>(has[rb] ? ks[rb] - 4 * h : 0);
    w[10 + rb] = static_cast<uint32_t>(has[rb] ? ke[rb] - ks[rb] : 0);
  }
  // Transposing reads of K^T (see read_xt): address of head_dim block db,
  // read a, ring slot 0, k-step 0.
  const int tj = (lane >> 2) & 3, tq = lane & 3, tdh = (lane >> 4) & 1;
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int row = 8 * a + 4 * h + tj;
    const int clo = 2 * tdh + (tq >> 1);
    const uint32_t toff = lds0 + row * kRowBytes + ((clo ^ ((row >> 2) & 3)) << 4) + ((tq & 1) << 3);
#pragma unroll
    for (int db = 0; db < 4; ++db) w[12 + 2 * db + a] = toff + (((db ^ tj) & 3) << 6);
  }
  // DMA offsets (16 key rows per wave, four rows per load) and the K row
  // read address of k-step 0 (the loop XORs in 32 kk).
  const uint32_t krowbytes = static_cast<uint32_t>(p.hkv) * kRowBytes;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * wave + 4 * i + (lane >> 4);
    const int j = (lane & 15) ^ swz(row);
    w[20 + i] = static_cast<uint32_t>(row) * krowbytes + 16 * j;
  }
  w[24] = lds0 + n * kRowBytes + ((h ^ swz(n)) << 4);
  w[25] = w[26] = w[27] = 0;
  {
    uint4* aux = reinterpret_cast<uint4*>(smem + dq_aux_offset(wave) + 16 * lane);
    // groups as the loop reads them: 0 dq / Q offsets, 1 -LSE / Delta, 2
    // row bounds, 3-4 transposing read addresses, 5 DMA offsets, 6 K read
    // address
#pragma unroll
    for (int g = 0; g < kDqAuxGroups; ++g)
      aux[64 * g] = make_uint4(w[4 * g], w[4 * g + 1], w[4 * g + 2], w[4 * g + 3]);
  }

  const uint64_t kvoff = static_cast<uint64_t>(kvh) * kRowBytes +
                         static_cast<uint64_t>(t_begin) * kBN * krowbytes;
  const uint64_t kbase = reinterpret_cast<uint64_t>(p.k) + kvoff;
  const uint64_t vbase = reinterpret_cast<uint64_t>(p.v) + kvoff;
  // Bytes of K (and V) from the item's first tile to the end of its last
  // tile or of the keys, whichever comes first (below 2^31: use_dq_wide).
  const int64_t krows = min(static_cast<int64_t>(p.total_kv) - static_cast<int64_t>(t_begin) * kBN,
                            static_cast<int64_t>(n_tiles) * kBN);
  const int kbytes = static_cast<int>(max(krows, int64_t{0}) * krowbytes);
  const uint32_t qbytes = static_cast<uint32_t>(p.total_q) * static_cast<uint32_t>(p.hq) * kRowBytes;
  const i32x4 qrsrc = make_rsrc(p.q, qbytes);
  const i32x4 dorsrc = make_rsrc(p.dout, qbytes);
  const i32x4 dqrsrc = make_rsrc(p.dq, qbytes);
  // This wave's pieces partials: units of row blocks 2 wave and 2 wave + 1.
  const char* part = reinterpret_cast<const char*>(p.dq_part) +
                     (static_cast<int64_t>(blockIdx.x) * kBwdWaves + 2 * wave) * kDqPartUnits * 1024;
  const i32x4 prsrc = make_rsrc(piece ? part : reinterpret_cast<const char*>(p.dq), piece ? 2 * kDqPartUnits * 1024 : 0);
  const uint32_t kb_lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(kbase));
  const uint32_t kb_hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(kbase >> 32));
  const uint32_t vb_lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(vbase));
  const uint32_t vb_hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(vbase >> 32));
  const uint64_t kb64 = (static_cast<uint64_t>(kb_hi) << 32) | kb_lo;
  const uint64_t vb64 = (static_cast<uint64_t>(vb_hi) << 32) | vb_lo;
  const float c = p.c, scale = p.scale;
  asm volatile(SWATTN_BWD_DQ_ASM
               :
               : [kbase] "s"(kb64), [vbase] "s"(vb64), [qrsrc] "s"(qrsrc), [dorsrc] "s"(dorsrc),
                 [dqrsrc] "s"(dqrsrc), [prsrc] "s"(prsrc),
                 [ntiles] "s"(__builtin_amdgcn_readfirstlane(n_tiles)),
                 [kbytes] "s"(__builtin_amdgcn_readfirstlane(kbytes)),
                 [ktilebytes] "s"(__builtin_amdgcn_readfirstlane(static_cast<int>(kBN * krowbytes))),
                 [key0] "s"(__builtin_amdgcn_readfirstlane(t_begin * kBN)),
                 [it0] "s"(__builtin_amdgcn_readfirstlane(it0)),
                 [it1] "s"(__builtin_amdgcn_readfirstlane(it1)), [c] "s"(c), [scale] "s"(scale),
                 [ldsw] "s"(__builtin_amdgcn_readfirstlane(lds0 + wave * 4096)),
                 [aux] "s"(__builtin_amdgcn_readfirstlane(lds0 + dq_aux_offset(wave))),
                 [ebase] "s"(__builtin_amdgcn_readfirstlane(lds0 + wave * SWATTN_BWD_DQ_EPI_REGION)),
                 [piece] "s"(__builtin_amdgcn_readfirstlane(piece ? 1 : 0))
               : SWATTN_BWD_DQ_CLOBBERS);
}

// dQ of row tiles cut into pieces: one thread per (row tile and KV head,
// wave, float4 unit, lane); row tiles left whole were stored by the dQ
// kernel.  It sums that unit over the pieces in piece order
// (deterministic) and stores its four bf16 values where a whole row tile
// would: the lane's row of the tile, d-rows 32d + 8j + 4h .. +3.
static_assert(kDqPartUnits == 16 && kBwdWaves == 8, "the reduce's thread index splits 6 + 4 + 3 bits");
__global__ __launch_bounds__(kThreads) void bwd_dq_reduce_kernel(const BwdParams p) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int lane = static_cast<int>(id & 63);
  const int u = static_cast<int>((id >> 6) & (kDqPartUnits - 1));
  const int wave = static_cast<int>((id >> 10) & (kBwdWaves - 1));
  const int tk = static_cast<int>(id >> 13);   // (row tile t, KV head), KV head fastest
  const int kvh = tk % p.hkv, t = tk / p.hkv;
  const int nch = p.dq_nch[tk];
  if (nch <= 1) return;
  // The row tile's first workgroup slot (slots are ordered as the dQ grid).
  const int64_t slot0 = t < p.items[0]
                            ? static_cast<int64_t>(t) * p.dq_maxc[0]
                            : static_cast<int64_t>(p.items[0]) * p.dq_maxc[0] +
                                  static_cast<int64_t>(t - p.items[0]) * p.dq_maxc[1];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp = 0; sp < nch; ++sp) {
    const int64_t wg = (slot0 + sp) * p.hkv + kvh;
    const float4 a = *dq_part_unit(p, wg, wave, u, lane);
    acc.x += a.x;
    acc.y += a.y;
    acc.z += a.z;
    acc.w += a.w;
  }
  const int b = t < p.items[0] ? 0 : 1;
  const int item = b == 0 ? p.items[0] - 1 - t : p.items[0] + p.items[1] - 1 - t;
  const int blk = item * (kRowsPerItem / kBRows) + wave;
  const int r = blk * kBRows + (lane & 31);
  if (blk >= p.blocks[b] || r >= p.nrows[b]) return;
  const int G = p.group;
  const int q_slot = r / G;
  const int pos = p.idx[b][q_slot];
  if (!pos_ok(p, pos)) return;
  const int qh = kvh * G + (r - q_slot * G);
  const int d = u >> 2, j = u & 3;
  uint2 w;
  w.x = pack_bf16x2(acc.x * p.scale, acc.y * p.scale);
  w.y = pack_bf16x2(acc.z * p.scale, acc.w * p.scale);
  *reinterpret_cast<uint2*>(p.dq + (static_cast<int64_t>(pos) * p.hq + qh) * kD +
                            4 * (lane >> 5) + 32 * d + 8 * j) = w;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct BwdLayout {
  int64_t blocks[2], items[2], total_blocks, kv_tiles_dkv, dkv_split, dq_chunk, dq_maxc[2];
  size_t off_info, off_zero, off_ranges, off_part, off_dq_nch, off_dq_part, bytes;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// bwd_dq_wide_kernel addresses Q, dO, dq and the item's K / V bytes with
// 32-bit buffer offsets (and drops out-of-range ones): both must stay below
// 2^31 bytes.  SWATTN_DQ_KERNEL=narrow / wide picks a kernel for tests and
// comparisons.
// bwd_dkdv_wide_kernel gathers rows by 32-bit offsets into Q / dO and reads
// K, V, dK, dV and the row info through 32-bit buffer ranges (all below
// 2^31 bytes).  It runs split or unsplit, as the layout decides;
// SWATTN_DKDV_KERNEL=narrow picks the eight-wave kernel (tests and
// comparisons).
inline bool use_dkdv_wide(int64_t total_q, int64_t total_kv, int32_t heads_q, int32_t heads_kv,
                          int64_t total_blocks) {
  if (total_q * heads_q * kRowBytes >= (int64_t{1} << 31)) return false;
  if (total_kv * heads_kv * kRowBytes >= (int64_t{1} << 31)) return false;
  if (total_blocks * kInfoBytes >= (int64_t{1} << 31)) return false;
  const char* force = getenv("SWATTN_DKDV_KERNEL");
  if (force != nullptr && strcmp(force, "narrow") == 0) return false;
  return true;
}

inline bool use_dq_wide(int64_t total_q, int64_t total_kv, int32_t heads_q, int32_t heads_kv) {
  if (total_q * heads_q * kRowBytes >= (int64_t{1} << 31)) return false;
  if (total_kv * heads_kv * kRowBytes >= (int64_t{1} << 31)) return false;
  const char* force = getenv("SWATTN_DQ_KERNEL");
  if (force != nullptr && strcmp(force, "narrow") == 0) return false;
  return true;
}

inline BwdLayout bwd_layout(int64_t seq_kv, int64_t total_kv, int32_t heads_kv, int64_t group,
                            int32_t window, int64_t n_full, int64_t n_local) {
  BwdLayout L{};
  const int64_t n[2] = {n_full, n_local};
  for (int b = 0; b < 2; ++b) {
    L.blocks[b] = ceil_div(n[b] * group, kBRows);
    L.items[b] = ceil_div(n[b] * group, kRowsPerItem);
  }
  L.total_blocks = static_cast<int64_t>(heads_kv) * (L.blocks[0] + L.blocks[1]);
  L.kv_tiles_dkv = ceil_div(total_kv, kKeysDkv);
  // Fewer (key tile, KV head) pairs than two rounds of workgroups: each pair
  // is split over its row blocks, so that the longest pair (the first key
  // tile sees every full row) no longer sets the kernel's length.
  const int64_t pairs = L.kv_tiles_dkv * heads_kv;
  L.dkv_split = pairs >= kDkvTargetWgs ? 1
                : std::min<int64_t>(kDkvMaxSplit, ceil_div(kDkvTargetWgs, pairs));
  size_t o = 0;
  L.off_info = o;   o = align256(o + static_cast<size_t>(L.total_blocks) * kInfoBytes);
  L.off_zero = o;   o = align256(o + kRowBytes);
  L.off_ranges = o; o = align256(o + static_cast<size_t>(2 * L.kv_tiles_dkv) * 2 * sizeof(int32_t));
  L.off_part = o;
  if (L.dkv_split > 1) o += static_cast<size_t>(pairs * L.dkv_split) * kPartBytesPerWg;
  // dQ: a row tile's key tiles, estimated per branch (a full row tile of
  // one sequence spans up to a sequence's keys, half of them on average; a
  // local one about a window).  When the longest one exceeds the estimated
  // tiles per workgroup slot (the sum over kDqSlots slots), row tiles are
  // cut into pieces of at most that many tiles (at least
  // kDqMinTilesPerPiece), so that the longest no longer sets the kernel's
  // length.  (Measured on the KV-head share of a 16K-token, 4-query-head
  // prefill: pieces of 0.5x, 0.625x, 0.75x, 1.5x and 2x the per-slot tiles
  // all ran 5-15% slower than 1x.)  Each row tile has room for as many
  // pieces as its branch's longest estimate needs.
  const int64_t q_items = (L.items[0] + L.items[1]) * heads_kv;
  const int64_t full_len = ceil_div(seq_kv, kBN) + 1;
  const int64_t local_len = std::min<int64_t>(full_len, ceil_div(window, kBN) + 2);
  const int64_t est = heads_kv * (L.items[0] * (full_len / 2 + 1) + L.items[1] * local_len);
  const int64_t per_slot = ceil_div(est, kDqSlots);
  const int64_t longest = L.items[0] > 0 ? full_len : local_len;
  L.dq_chunk = 0;
  L.dq_maxc[0] = L.dq_maxc[1] = 1;
  if (q_items > 0 && longest > per_slot && longest > kDqMinTilesPerPiece) {
    L.dq_chunk = std::max<int64_t>(kDqMinTilesPerPiece, per_slot);
    L.dq_maxc[0] = ceil_div(full_len, L.dq_chunk);
    L.dq_maxc[1] = ceil_div(local_len, L.dq_chunk);
  }
  // Partials are indexed by the dQ workgroup; full row tiles' slots come
  // first, and local ones are only cut when their branch has more than one
  // slot.  With the rule above a branch can be cut only if it has fewer than
  // 512 (full) or 256 (local) row tiles times KV heads, and their pieces
  // number at most 512 or 256 more than that: under 1024 full and 512 local
  // slots, 192 MiB.
  L.off_dq_nch = o;
  L.off_dq_part = o;
  if (L.dq_chunk > 0) {
    o = align256(o + static_cast<size_t>(q_items) * sizeof(int32_t));
    L.off_dq_part = o;
    const int64_t slots = L.items[0] * L.dq_maxc[0] + (L.dq_maxc[1] > 1 ? L.items[1] * L.dq_maxc[1] : 0);
    o += static_cast<size_t>(heads_kv * slots) * kDqPartBytesPerWg;
  }
  L.bytes = o;
  return L;
}

}  // namespace
}  // namespace swattn

using namespace swattn;
using namespace swattn::tiles;

extern "C" size_t swattn_prefill_bwd_workspace_bytes(int32_t batch, int64_t seq_kv,
                                                     int32_t heads_q, int32_t heads_kv,
                                                     int32_t head_dim, int32_t window,
                                                     int64_t n_full, int64_t n_local) {
  if (batch < 1 || seq_kv < 1 || heads_q < 1 || heads_kv < 1 || head_dim != kD ||
      heads_q % heads_kv != 0 || window <= 0 || n_full < 0 || n_local < 0)
    return 0;
  const BwdLayout L = bwd_layout(seq_kv, static_cast<int64_t>(batch) * seq_kv, heads_kv,
                                 heads_q / heads_kv, window, n_full, n_local);
  return L.bytes;
}

extern "C" int swattn_prefill_bwd(const void* q, const void* k, const void* v, const void* out,
                                  const float* lse, const void* dout, const int32_t* full_idx,
                                  int64_t n_full, const int32_t* local_idx, int64_t n_local,
                                  const int32_t* full_starts, const int32_t* local_starts,
                                  const int32_t* causal_ends, void* dq, void* dk, void* dv,
                                  int32_t batch, int64_t seq_q, int64_t seq_kv, int32_t heads_q,
                                  int32_t heads_kv, int32_t head_dim, int32_t window,
                                  float scale_log2, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  if (head_dim != kD) return invalid("swattn_prefill_bwd: head_dim must be 128");
  if (batch < 1 || seq_q < 0 || seq_kv < 1 || heads_q < 1 || heads_kv < 1)
    return invalid("swattn_prefill_bwd: bad shape");
  if (heads_q % heads_kv != 0)
    return invalid("swattn_prefill_bwd: heads_q must be a multiple of heads_kv");
  // Per-lane staging offsets inside a key tile are 32-bit: (rows of a tile) x
  // heads_kv x 256 bytes must stay below 2^31.
  if (heads_kv > 4096 || heads_q > 65536)
    return invalid("swattn_prefill_bwd: at most 4096 KV heads and 65536 query heads");
  if (window <= 0) return invalid("swattn_prefill_bwd: window must be positive");
  if (!(scale_log2 > 0.f) || !isfinite(scale_log2))
    return invalid("swattn_prefill_bwd: scale_log2 must be positive and finite");
  if (n_full < 0 || n_local < 0 || n_full + n_local > static_cast<int64_t>(batch) * seq_q)
    return invalid("swattn_prefill_bwd: bad index counts");
  const int64_t total_q = static_cast<int64_t>(batch) * seq_q;
  const int64_t total_kv = static_cast<int64_t>(batch) * seq_kv;
  if (total_q > INT32_MAX || total_kv > INT32_MAX - 2 * kKeysDkv)
    return invalid("swattn_prefill_bwd: batch*seq must stay below 2^31");
  const int64_t group = heads_q / heads_kv;
  if ((n_full + n_local) * group > INT32_MAX - kRowsPerItem)
    return invalid("swattn_prefill_bwd: too many rows");
  const bool meta = full_starts != nullptr || local_starts != nullptr || causal_ends != nullptr;
  if (meta && (full_starts == nullptr || local_starts == nullptr || causal_ends == nullptr))
    return invalid("swattn_prefill_bwd: metadata needs full_starts, local_starts and causal_ends");
  // dk / dv are written for every key even without query rows (as zeros);
  // the row-side buffers are only needed when there are rows.
  if (k == nullptr || v == nullptr || dk == nullptr || dv == nullptr)
    return invalid("swattn_prefill_bwd: null pointer");
  if (n_full + n_local > 0 &&
      (q == nullptr || out == nullptr || lse == nullptr || dout == nullptr || dq == nullptr ||
       (n_full > 0 && full_idx == nullptr) || (n_local > 0 && local_idx == nullptr)))
    return invalid("swattn_prefill_bwd: null pointer");
  if (!aligned16(k) || !aligned16(v) || !aligned16(dk) || !aligned16(dv) ||
      (n_full + n_local > 0 &&
       (!aligned16(q) || !aligned16(out) || !aligned16(dout) || !aligned16(dq))))
    return invalid("swattn_prefill_bwd: q, k, v, out, dout, dq, dk and dv must be 16-byte aligned");
  const BwdLayout L = bwd_layout(seq_kv, total_kv, heads_kv, group, window, n_full, n_local);
  if (workspace == nullptr || workspace_bytes < L.bytes) {
    set_error("swattn_prefill_bwd: workspace smaller than swattn_prefill_bwd_workspace_bytes()");
    return SWATTN_EWORKSPACE;
  }
  if (!aligned256(workspace)) return invalid("swattn_prefill_bwd: workspace must be 256-byte aligned");
  if (L.kv_tiles_dkv * heads_kv * L.dkv_split > INT32_MAX ||
      (L.items[0] * L.dq_maxc[0] + L.items[1] * L.dq_maxc[1]) * heads_kv > INT32_MAX ||
      (L.dq_chunk > 0 &&
       (L.items[0] + L.items[1]) * heads_kv * kBwdWaves * kDqPartUnits * 64 / kThreads > INT32_MAX))
    return invalid("swattn_prefill_bwd: grid too large");

  char* ws = static_cast<char*>(workspace);
  BwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<const uint16_t*>(out);
  p.dout = static_cast<const uint16_t*>(dout);
  p.lse = lse;
  p.dq = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.idx[0] = full_idx;
  p.idx[1] = local_idx;
  p.starts[0] = full_starts;
  p.starts[1] = local_starts;
  p.ends = causal_ends;
  p.count[0] = static_cast<int32_t>(n_full);
  p.count[1] = static_cast<int32_t>(n_local);
  for (int b = 0; b < 2; ++b) {
    p.nrows[b] = static_cast<int32_t>(p.count[b] * group);
    p.blocks[b] = static_cast<int32_t>(L.blocks[b]);
    p.items[b] = static_cast<int32_t>(L.items[b]);
  }
  p.blk_base[0] = 0;
  p.blk_base[1] = static_cast<int64_t>(heads_kv) * L.blocks[0];
  p.info = ws + L.off_info;
  p.zero_row = reinterpret_cast<uint16_t*>(ws + L.off_zero);
  p.ranges = reinterpret_cast<int32_t*>(ws + L.off_ranges);
  p.seq_q = static_cast<int32_t>(seq_q);
  p.seq_kv = static_cast<int32_t>(seq_kv);
  p.total_q = static_cast<int32_t>(total_q);
  p.total_kv = static_cast<int32_t>(total_kv);
  p.kv_tiles_dkv = static_cast<int32_t>(L.kv_tiles_dkv);
  p.dkv_split = static_cast<int32_t>(L.dkv_split);
  // Several sequences that each hold whole 256-key tiles: interleave them.
  p.dkv_batches = (batch > 1 && seq_kv % kKeysDkv == 0) ? batch : 1;
  p.dkv_part = reinterpret_cast<float*>(ws + L.off_part);
  p.dq_chunk = static_cast<int32_t>(L.dq_chunk);
  p.dq_maxc[0] = static_cast<int32_t>(L.dq_maxc[0]);
  p.dq_maxc[1] = static_cast<int32_t>(L.dq_maxc[1]);
  p.dq_nch = reinterpret_cast<int32_t*>(ws + L.off_dq_nch);
  p.dq_part = reinterpret_cast<float*>(ws + L.off_dq_part);
  p.hq = heads_q;
  p.hkv = heads_kv;
  p.group = static_cast<int32_t>(group);
  p.window = window;
  p.c = scale_log2;
  p.scale = scale_log2 * 0.69314718055994531f;   // sm_scale = c * ln 2

  const hipStream_t st = as_stream(stream);
  const uint32_t rgrid = static_cast<uint32_t>(ceil_div(2 * L.kv_tiles_dkv, kThreads / 64));
  if (meta)
    hipLaunchKernelGGL(bwd_ranges_kernel<true>, dim3(rgrid), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(bwd_ranges_kernel<false>, dim3(rgrid), dim3(kThreads), 0, st, p);
  const int64_t nblk = L.blocks[0] + L.blocks[1];
  if (nblk > 0) {
    if (meta)
      hipLaunchKernelGGL(bwd_prep_kernel<true>, dim3(static_cast<uint32_t>(nblk), heads_kv),
                         dim3(kThreads), 0, st, p);
    else
      hipLaunchKernelGGL(bwd_prep_kernel<false>, dim3(static_cast<uint32_t>(nblk), heads_kv),
                         dim3(kThreads), 0, st, p);
  }
  const int64_t pairs = L.kv_tiles_dkv * heads_kv;
  const bool dkdv_wide = use_dkdv_wide(total_q, total_kv, heads_q, heads_kv, L.total_blocks);
  if (dkdv_wide)
    hipLaunchKernelGGL(bwd_dkdv_wide_kernel, dim3(static_cast<uint32_t>(pairs * L.dkv_split)), dim3(256), 0,
                       st, p);
  else
    hipLaunchKernelGGL(bwd_dkdv_kernel, dim3(static_cast<uint32_t>(pairs * L.dkv_split)),
                       dim3(kBwdThreads), 0, st, p);
  if (L.dkv_split > 1)
    hipLaunchKernelGGL(bwd_dkdv_reduce_kernel,
                       dim3(static_cast<uint32_t>(pairs * kBwdWaves * kPartUnits * 64 / kThreads)),
                       dim3(kThreads), 0, st, p);
  const int64_t q_items = (L.items[0] + L.items[1]) * heads_kv;
  if (q_items > 0) {
    const int64_t dq_wgs = (L.items[0] * L.dq_maxc[0] + L.items[1] * L.dq_maxc[1]) * heads_kv;
    if (use_dq_wide(total_q, total_kv, heads_q, heads_kv))
      hipLaunchKernelGGL(bwd_dq_wide_kernel, dim3(static_cast<uint32_t>(dq_wgs)), dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL(bwd_dq_kernel, dim3(static_cast<uint32_t>(dq_wgs)), dim3(kBwdThreads), 0,
                         st, p);
    if (L.dq_chunk > 0)
      hipLaunchKernelGGL(bwd_dq_reduce_kernel,
                         dim3(static_cast<uint32_t>(q_items * kBwdWaves * kDqPartUnits * 64 / kThreads)),
                         dim3(kThreads), 0, st, p);
  }
  return launch_status("swattn_prefill_bwd");
}
