// Tile building blocks shared by the paged decode and prefill kernels
// (gfx950, wave64 + MFMA): 16-token K/V tiles staged in LDS by direct
// HBM -> LDS copies under an XOR piece swizzle, the S^T = K Q^T and
// O += P V MFMA tile updates, and exact vmcnt waits.
#pragma once

#include "mv_common.h"

namespace mv {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kTile = 16;       // tokens per K/V tile (MFMA M of S^T)
constexpr int kMaxGroup = 16;   // MFMA N: query rows per tile
constexpr float kNegInf = -__builtin_huge_valf();

// Geometry of one 16-token tile of one head.
template <int DTYPE, int D>
struct TileGeom {
  static constexpr int kElemBytes = Elem<DTYPE>::bytes;
  static constexpr int kRowBytes = D * kElemBytes;     // one token row of one head
  static constexpr int kTileBytes = kTile * kRowBytes;  // 2 KiB (D=64, 16-bit) .. 8 KiB
  static constexpr int kLoads = kTileBytes / 1024;      // 1 KiB load instructions per tile
  static constexpr int kRowPieces = kRowBytes / 16;     // 16-byte pieces per row: 8, 16, 32
  static constexpr int kLaneElems = D / 4;              // MFMA: dims per lane per token
  static constexpr int kLanePieces = kLaneElems * kElemBytes / 16;
  static constexpr int kElemsPerPiece = 16 / kElemBytes;
};

// Swizzle of the 16-byte pieces of LDS row r (r < 16): slot s holds piece
// s ^ sw(r). sw is the XOR of row bits that makes both reads of a tile
// free of bank conflicts, whether the LDS serves 32 or 64 banks of 4 bytes
// a cycle (found by an exhaustive search over such swizzles against a bank
// model of the two reads):
//   * the K-operand read, ds_read_b128: lane (g, t) reads row t, piece
//     g * kLanePieces + c;
//   * the transposed V read, ds_read_b64_tr_b16: lane (g, t) reads 8 bytes
//     of row 4g + t/4, piece 2c + (t%4)/2 (v_column_tr below).
// 8 pieces (head_dim 64, 16-bit): bits (r2, r1, r0^r2^r3); 16 pieces
// (head_dim 128 16-bit, head_dim 64 fp32): bits (r2, r0, r1, r2^r3). The
// earlier (r >> 1) & 7 and r & 15 left the V reads 2-way (64 banks) and 4-way
// (32 banks) conflicted.
template <int ROW_PIECES>
__device__ __forceinline__ int piece_swizzle(int r) {
  if constexpr (ROW_PIECES == 8)
    return ((r >> 2) & 1) | (r & 2) | (((r ^ (r >> 2) ^ (r >> 3)) & 1) << 2);
  else if constexpr (ROW_PIECES == 16)
    return ((r >> 2) & 1) | ((r & 1) << 1) | ((r & 2) << 1) | ((((r >> 2) ^ (r >> 3)) & 1) << 3);
  else
    return r & 15;
}

// S^T tile update: acc += K(16 tokens x 32 dims) * Q^T(32 dims x 16 heads)
// for the 16-bit types; one call per 16-byte piece of the lane's dims.
template <int DTYPE>
__device__ __forceinline__ f32x4 mfma_qk(const uint4& k, const uint4& q, f32x4 acc);
template <>
__device__ __forceinline__ f32x4 mfma_qk<MV_DTYPE_BF16>(const uint4& k, const uint4& q, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, k),
                                                  __builtin_bit_cast(bf16x8, q), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_qk<MV_DTYPE_F16>(const uint4& k, const uint4& q, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, k),
                                                 __builtin_bit_cast(f16x8, q), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_qk<MV_DTYPE_F32>(const uint4& k, const uint4& q, f32x4 acc) {
  // 4 dims per 16-byte piece, one 16x16x4 fp32 MFMA per dim slot.
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(k.x), __uint_as_float(q.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(k.y), __uint_as_float(q.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(k.z), __uint_as_float(q.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(k.w), __uint_as_float(q.w), acc, 0, 0, 0);
  return acc;
}

// acc + the dot product of two 16-byte pieces (8 16-bit or 4 fp32 elements)
// on the VALU: v_dot2 with fp32 accumulation for the 16-bit types, plain
// FMAs for fp32.
template <int DTYPE>
__device__ __forceinline__ float dot_piece(const uint4& a, const uint4& b, float acc) {
  const uint32_t x[4] = {a.x, a.y, a.z, a.w}, y[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DTYPE == MV_DTYPE_BF16) {
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x[i]),
                                             __builtin_bit_cast(bf16x2_t, y[i]), acc, false);
    } else if constexpr (DTYPE == MV_DTYPE_F16) {
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x[i]), __builtin_bit_cast(f16x2_t, y[i]),
                                   acc, false);
    } else {
      acc = fmaf(__uint_as_float(x[i]), __uint_as_float(y[i]), acc);
    }
  }
  return acc;
}

// V elements (row 4g+e, column 16c+t), e = 0..3, of a swizzled 16-bit LDS
// tile in one instruction: gfx950's transposed LDS read. Within each group
// of 16 lanes, lane i receives halfword (i % 4) of the 8 bytes that lane
// 4e + i / 4 of the group addresses, for e = 0..3 (lane layout measured on
// the hardware with an in-bounds probe). Lane (g, t) therefore addresses
// row 4g + t/4 at columns 16c + 4(t%4) .. +3 and gets column 16c+t of rows
// 4g..4g+3 -- the B operand of a 16x16x16 MFMA with K = tokens.
template <int RP>
__device__ __forceinline__ s16x4 v_column_tr(const char* v_tile, int g, int t, int c) {
  const int row = 4 * g + (t >> 2);
  const int col = 16 * c + 4 * (t & 3);  // halfword column, 8-byte aligned
  const int piece = col >> 3;            // 8 halfwords per 16-byte piece
  const char* src = v_tile + row * RP * 16 + ((piece ^ piece_swizzle<RP>(row)) << 4) + ((col & 7) << 1);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(const_cast<char*>(src)));
}

// Max / sum over the four 16-lane rows of the wave (lanes t, t+16, t+32,
// t+48: one MFMA result column), every lane receiving the result, in two
// gfx950 permlane swaps (VALU) instead of two LDS permutes. permlane32_swap
// of (x, x) yields (rows 0 1 0 1, rows 2 3 2 3), permlane16_swap yields
// (rows 0 0 2 2, rows 1 1 3 3); combining each pair reduces over row bits
// 1, then 0. Used by the decode tile loop (c2 layer call 1 % faster);
// the prefill, bound by VALU issue, keeps the LDS permutes (3 % faster
// there).
__device__ __forceinline__ float rows_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// The value lane ^ 32 holds (the other half of the wave), for 16 bytes per
// lane: one permlane32 swap per dword (VALU, no LDS). permlane32_swap of
// (x, x) yields (rows 0 1 0 1, rows 2 3 2 3) as above, so lanes 0-31 find
// lanes 32-63's values in the second result and lanes 32-63 lanes 0-31's
// in the first.
__device__ __forceinline__ uint32_t swap_wave_halves_u32(uint32_t x, int lane) {
  const auto a = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return (lane & 32) ? a[0] : a[1];
}
__device__ __forceinline__ uint4 swap_wave_halves(uint4 x, int lane) {
  return make_uint4(swap_wave_halves_u32(x.x, lane), swap_wave_halves_u32(x.y, lane),
                    swap_wave_halves_u32(x.z, lane), swap_wave_halves_u32(x.w, lane));
}

// P values of one lane (4 per 16-token tile, fp32) rounded to the 16-bit
// MFMA input type in two packed conversions, returned as the PV MFMA's A
// operand; `sum` accumulates the rounded values (two dot2 with (1, 1)), so
// O / l stays an exact convex combination of V rows.
template <int DTYPE>
__device__ __forceinline__ s16x4 pack_p(float p0, float p1, float p2, float p3, float& sum) {
  static_assert(DTYPE != MV_DTYPE_F32, "16-bit types only");
  uint32_t lo, hi;
  if constexpr (DTYPE == MV_DTYPE_BF16) {
    const bf16x2_t a = __builtin_convertvector((f32x2_t){p0, p1}, bf16x2_t);
    const bf16x2_t b = __builtin_convertvector((f32x2_t){p2, p3}, bf16x2_t);
    const bf16x2_t ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
    sum = __builtin_amdgcn_fdot2_f32_bf16(a, ones, sum, false);
    sum = __builtin_amdgcn_fdot2_f32_bf16(b, ones, sum, false);
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
  } else {
    const f16x2_t a = __builtin_convertvector((f32x2_t){p0, p1}, f16x2_t);
    const f16x2_t b = __builtin_convertvector((f32x2_t){p2, p3}, f16x2_t);
    const f16x2_t ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
    sum = __builtin_amdgcn_fdot2(a, ones, sum, false);
    sum = __builtin_amdgcn_fdot2(b, ones, sum, false);
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
  }
  return __builtin_bit_cast(s16x4, make_uint2(lo, hi));
}

// The transposed V operands of one 16-token tile (16-bit types), one per
// 16-dim column block, for mfma_pv_operands.
template <int DTYPE, int D>
__device__ __forceinline__ void read_v_operands(const char* v_tile, int g, int t, s16x4 (&vb)[D / 16]) {
  constexpr int RP = TileGeom<DTYPE, D>::kRowPieces;
#pragma unroll
  for (int c = 0; c < D / 16; ++c) vb[c] = v_column_tr<RP>(v_tile, g, t, c);
}
// o[r][c] += P_r V from V operands already read (read_v_operands).
template <int DTYPE, int D, int R>
__device__ __forceinline__ void mfma_pv_operands(const s16x4 (&pa)[R], const s16x4 (&vb)[D / 16],
                                                 f32x4 (&o)[R][D / 16]) {
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (DTYPE == MV_DTYPE_BF16) {
        o[r][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa[r], vb[c], o[r][c], 0, 0, 0);
      } else {
        o[r][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, pa[r]),
                                                       __builtin_bit_cast(f16x4, vb[c]), o[r][c], 0, 0, 0);
      }
    }
  }
}

// o[r][c] += P_r V over two 16-token tiles a and b in one 16x16x32 MFMA per
// column block (16-bit types): K slots 8g..8g+3 are tile a's tokens 4g..4g+3
// and slots 8g+4..8g+7 tile b's, in both the P operand (pack_p of a, then b)
// and the V operand (transposed reads of a, then b).
template <int DTYPE, int D, int R>
__device__ __forceinline__ void mfma_pv2_operands(const s16x4 (&pa)[R], const s16x4 (&pb)[R],
                                                  const s16x4 (&va)[D / 16], const s16x4 (&vb)[D / 16],
                                                  f32x4 (&o)[R][D / 16]) {
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    const s16x8 v = __builtin_shufflevector(va[c], vb[c], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const s16x8 p = __builtin_shufflevector(pa[r], pb[r], 0, 1, 2, 3, 4, 5, 6, 7);
      if constexpr (DTYPE == MV_DTYPE_BF16) {
        o[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, p),
                                                          __builtin_bit_cast(bf16x8, v), o[r][c], 0, 0, 0);
      } else {
        o[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, p),
                                                         __builtin_bit_cast(f16x8, v), o[r][c], 0, 0, 0);
      }
    }
  }
}

// O tile update for one 16-token tile, 16-bit types, P already packed
// (pack_p): o[r][c] += P_r V for R row tiles that share the tile.
template <int DTYPE, int D, int R>
__device__ __forceinline__ void mfma_pv_packed(const s16x4 (&pa)[R], const char* v_tile, int g, int t,
                                               f32x4 (&o)[R][D / 16]) {
  constexpr int RP = TileGeom<DTYPE, D>::kRowPieces;
  // At head_dim 64 all of the tile's V operands are read before the first
  // MFMA, so the reads overlap each other instead of each MFMA waiting for
  // its own (the scheduler would sink them); at 128 the pinned reads would
  // not fit the prefill's registers, and the scheduler places them.
  s16x4 vb[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) vb[c] = v_column_tr<RP>(v_tile, g, t, c);
  if constexpr (D <= 64) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (DTYPE == MV_DTYPE_BF16) {
        o[r][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa[r], vb[c], o[r][c], 0, 0, 0);
      } else {
        o[r][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, pa[r]),
                                                       __builtin_bit_cast(f16x4, vb[c]), o[r][c], 0, 0, 0);
      }
    }
  }
}

// O tile update for one 16-token tile from its swizzled LDS tile, for R
// row tiles that share the tile: o[r][c] += P_r(16 rows x 16 tokens)
// V(16 tokens x 16 dims), V element (row 4g+e, column 16c+t) per lane.
template <int DTYPE, int D, int R>
__device__ __forceinline__ void mfma_pv_rows(const float (&p)[R][4], const char* v_tile, int g,
                                             int t, f32x4 (&o)[R][D / 16]) {
  using Tr = TileGeom<DTYPE, D>;
  constexpr int RP = Tr::kRowPieces;
  constexpr int EPP = Tr::kElemsPerPiece;
  if constexpr (DTYPE == MV_DTYPE_F32) {
    int row_base[4], row_sw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      row_base[e] = (4 * g + e) * RP * 16;
      row_sw[e] = piece_swizzle<RP>(4 * g + e);
    }
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const int col = 16 * c + t;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int off = row_base[e] + (((col / EPP) ^ row_sw[e]) << 4) + (col % EPP) * 4;
        const float vv = *reinterpret_cast<const float*>(v_tile + off);
#pragma unroll
        for (int r = 0; r < R; ++r)
          o[r][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r][e], vv, o[r][c], 0, 0, 0);
      }
    }
  } else {
    s16x4 pa[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) pa[r][e] = static_cast<short>(from_f32<DTYPE>(p[r][e]));
    mfma_pv_packed<DTYPE, D, R>(pa, v_tile, g, t, o);
  }
}

// One row tile: o[c] += P V.
template <int DTYPE, int D>
__device__ __forceinline__ void mfma_pv(const float (&p)[4], const char* v_tile, int g, int t,
                                        f32x4 (&o)[D / 16]) {
  mfma_pv_rows<DTYPE, D, 1>(reinterpret_cast<const float(&)[1][4]>(p), v_tile, g, t,
                            reinterpret_cast<f32x4(&)[1][D / 16]>(o));
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima): this
// wave's vector memory operations, stores included, are complete.
constexpr unsigned kWaitVmcnt0 = 0x0F70;

// s_waitcnt vmcnt(N), N <= 63 (expcnt and lgkmcnt at their maxima; vmcnt
// is split over bits [3:0] and [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
}

// Waits until at most R * PER vector memory instructions of this wave are
// outstanding, R <= RMAX (R is wave-uniform, the count an immediate).
template <int PER, int RMAX>
__device__ __forceinline__ void wait_vmcnt_groups(int r) {
  if constexpr (RMAX == 0) {
    wait_vmcnt<0>();
  } else {
    if (r >= RMAX) wait_vmcnt<PER * RMAX>();
    else wait_vmcnt_groups<PER, RMAX - 1>(r);
  }
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}

// HBM -> LDS copy of 16 bytes per lane: lane l's bytes land at LDS address
// lds_base + 16 l (lds_base wave-uniform, passed in M0). Written as inline
// asm on purpose: the compiler then does not see a pending LDS write and
// does not put a vmcnt(0) in front of every later LDS access (which would
// wait for the tiles still streaming into the other buffers); the tile loop
// counts these loads itself. The "memory" clobber keeps LDS accesses of the
// wave on their side of the copy.
__device__ __forceinline__ void copy_to_lds_16B(const char* src, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_base) : "memory");
}
// HBM -> LDS copy of 4 bytes per lane: lane l's bytes land at LDS address
// lds_base + 4 l (as above).
__device__ __forceinline__ void copy_to_lds_4B(const char* src, uint32_t lds_base) {
  asm volatile("global_load_lds_dword %0, off" ::"v"(src), "{m0}"(lds_base) : "memory");
}
// The same copy from a wave-uniform base address (SGPRs) plus this lane's
// 32-bit byte offset (global_load_lds_dwordx4 with saddr): no 64-bit
// address arithmetic per lane. `sbase` must be the same in every lane.
__device__ __forceinline__ void copy_to_lds_16B_sv(const char* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_base) : "memory");
}

// Scalar base plus lane offset, non-temporal (see the two copies below).
__device__ __forceinline__ void copy_to_lds_16B_sv_stream(const char* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "{m0}"(lds_base) : "memory");
}

// The same copy with the non-temporal hint (nt): for data read once per
// launch, such as the decode's K/V tiles. Measured on the decode kernel:
// 5 % (c2-sized batches) to 13 % (head_dim 128, long contexts) less time
// than the default policy; sc0 / sc1 on top of it change nothing. The
// prefill, whose K/V tiles are read by several query-tile groups, is
// unchanged by it and keeps the default.
__device__ __forceinline__ void copy_to_lds_16B_stream(const char* src, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(lds_base) : "memory");
}

template <int C>
struct IntC {
  static constexpr int value = C;
};

}  // namespace
}  // namespace mv
