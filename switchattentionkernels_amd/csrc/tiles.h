// Tile layouts and data movement shared by the gfx950 attention kernels
// (forward and backward): operand vector types, the LDS chunk swizzles, the
// key-permutation inside 16-key groups, raw buffer descriptors, the
// global -> LDS DMA (buffer-descriptor and per-lane gather forms), and the
// V^T (or K^T) tile packer.
#pragma once

#include "common.h"

namespace swattn {
namespace tiles {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;                               // head_dim
constexpr int kBN = 64;                               // keys per K/V tile
constexpr int kRowBytes = kD * 2;                     // 256-byte K rows, unpadded
constexpr int kVtRowBytes = kBN * 2;                  // 128-byte V^T rows (one d, 64 keys)
constexpr int kTileBytes = kBN * kRowBytes;           // one K or V^T tile: 16 KiB
static_assert(kD * kVtRowBytes == kTileBytes, "K and V^T tiles have the same size");
// s_waitcnt immediate (gfx9 layout) for vmcnt(0) with expcnt and lgkmcnt
// left unconstrained: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14.
constexpr int kWaitVmcnt0 = (0x7 << 4) | (0xF << 8);

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

// Raw buffer resource (gfx9 layout): 48-bit base, stride 0, num_records
// bytes, 32-bit data format.  Lanes whose offset is >= num_records read
// nothing, so one descriptor covers a tile that is cut short by the end of
// the sequence, and num_records = 0 turns every load off.
constexpr int kRsrcWord3 = 0x00020000;
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(a)));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  r[3] = kRsrcWord3;
  return r;
}

// 16 bytes per lane from buffer offset voff to LDS at lds_base + 16 * lane
// (buffer_load_dwordx4 ... lds; the LDS base goes through M0 and must be
// wave-uniform).  Issued as inline assembly so that the compiler's wait
// insertion does not treat it as a store that aliases every LDS read; the
// memory clobber keeps it in order with the LDS reads around it.
__device__ __forceinline__ void dma16(const i32x4& rsrc, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds_base)
               : "memory", "m0");
}
// 16 bytes per lane from the 64-bit global address src to LDS at lds_base +
// 16 * lane (global_load_lds_dwordx4, gfx950): a gather with one source row
// per lane and no 4 GiB window.  Issued and waited for like dma16.
__device__ __forceinline__ void dma16_gather(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// X [total_kv, Hkv, 128] -> X^T tiles [Hkv][kv_tiles][128][64]: row d of tile
// t holds X[64t + key][d] for the 64 keys of the tile, each 16-key group in
// perm16 order, zeros past total_kv.  One block per (tile, KV head); the tile
// is staged through LDS (padded rows) and written as coalesced 16-byte chunks.
// (Internal linkage: every source that includes this header gets its own.)
namespace {
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
}  // namespace

// Row store through LDS.  A wave holds a 32 x 128 tile in the MFMA
// accumulator layout (acc[d][4j + i] of lane (r = lane % 32, h = lane / 32)
// is row r, column 32d + 8j + 4h + i); written to memory directly, each
// store instruction would put 16 bytes into each of 32 rows.  Staged through
// the wave's LDS region (32 rows at a 272-byte stride, then 32 row offsets),
// each store instruction writes four whole 256-byte rows.  row_off is the
// element offset of this lane's row in out, or -1 to skip the row.  The wave
// reads back only what it wrote (its LDS operations complete in order); the
// caller makes sure nothing else uses the region meanwhile.
constexpr int kORowBytes = kRowBytes + 16;
constexpr int kStoreRegionBytes = 32 * kORowBytes + 32 * 8;
__device__ __forceinline__ void store_rows_via_lds(char* region, int64_t row_off,
                                                   const f32x16 (&acc)[4], float scale,
                                                   uint16_t* __restrict__ out, int lane) {
  const int r = lane & 31, h = lane >> 5;
  int64_t* offs = reinterpret_cast<int64_t*>(region + 32 * kORowBytes);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 u;
      u.x = pack_bf16x2(acc[d][4 * j + 0] * scale, acc[d][4 * j + 1] * scale);
      u.y = pack_bf16x2(acc[d][4 * j + 2] * scale, acc[d][4 * j + 3] * scale);
      *reinterpret_cast<uint2*>(region + r * kORowBytes + 2 * (32 * d + 8 * j + 4 * h)) = u;
    }
  }
  if (h == 0) offs[r] = row_off;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 4 * i + (lane >> 4), c = lane & 15;
    const int64_t off = offs[row];
    const uint4 v = *reinterpret_cast<const uint4*>(region + row * kORowBytes + 16 * c);
    if (off >= 0) *reinterpret_cast<uint4*>(out + off + 8 * c) = v;
  }
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace tiles
}  // namespace swattn
