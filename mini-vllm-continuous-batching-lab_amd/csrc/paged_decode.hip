// Paged-attention decode for gfx950 (MI355X), wave64 + MFMA.
//
// Math (AttentionBackendRef.decode_attention,
// mini_vllm/attention/paged_attention_ref.py:102-161):
//   out[b, hq] = softmax(scale * q[b, hq] . K_b[hk]^T) V_b[hk],
//   hk = hq / n_rep, n_rep = Hq / Hkv (repeat_interleave grouping),
//   token j of sequence b at block_table[b, j / BS], offset j % BS.
//
// Work decomposition
//   Every sequence's context is cut into partitions of P tokens (P is
//   chosen per step by the plan kernel, a multiple of the chunk below). One
//   work group of kWaves wavefronts handles one (sequence, kv head,
//   partition) and serves all n_rep query heads of the GQA group, so every
//   K/V byte is read from HBM exactly once. The work group walks its
//   partition in chunks of kWaves 16-token tiles, one tile per wave.
//
// Per tile (16 tokens x D) and wave, with lane = 16*g + t (g = 0..3):
//   * HBM -> LDS without registers: global_load_lds_dwordx4 writes lane l's
//     16 bytes to LDS slot (64c + l) of load instruction c. Each lane
//     fetches the 16-byte piece that belongs in its slot under an XOR
//     swizzle (slot s of row r holds piece s ^ sw(r)), so every load
//     instruction still reads 1 KiB of contiguous HBM while the reads
//     below are bank-conflict free with unpadded rows. Two LDS buffers per
//     wave: the next tile streams in while the current one is computed.
//   * S^T = K Q^T on MFMA (16x16x32 for 16-bit types, 16x16x4 for fp32):
//     A = K tile (M = tokens), row t, dims [g*D/4, (g+1)*D/4) from LDS;
//     B = Q^T (N = query heads of the group, rows >= n_rep zero) from
//     registers. Both operands use the same k-slot -> dim mapping, so the
//     contraction covers all D dims whatever the hardware's k order.
//   * The accumulator holds S^T[token 4g+e][head t] in lane (g, t), slot e
//     -- the A-operand layout of the P V MFMA (M = heads, K = tokens), so
//     the probabilities never leave registers.
//   * V needs K = tokens in each lane: it is read from its LDS tile
//     column-wise.
//   Softmax is online across tiles (one rescale per tile) and exact within
//   a tile. The kWaves wave results are merged through LDS.
//
// Cross-partition merge (fused): a sequence with one partition writes the
// output directly. Otherwise each work group writes its normalised partial
// (o, max, sum) in fp32 with device-coherent stores, waits for them to
// complete and bumps the (sequence, kv head) counter; the work group that
// brings the counter to n_parts merges all partials with a log-sum-exp
// reduce (device-coherent loads), writes the output and resets the counter
// to zero. (A __threadfence() here would write back and invalidate the
// whole L2 of the XCD in every wave, which costs ~10x the kernel.)
// Counters are zeroed by the plan kernel, so every call that shares a plan
// must run on one stream.
#include <algorithm>
#include <climits>

#include "mv_common.h"

namespace mv {
namespace {

// Launch geometry (build-time tunables; the defaults are the shipped shape).
#ifndef MV_DECODE_WAVES
#define MV_DECODE_WAVES 4
#endif
constexpr int kWaves = MV_DECODE_WAVES;
constexpr int kTile = 16;
constexpr int kMaxGroup = 16;   // MFMA N: query heads per kv head
constexpr int kMaxParts = 128;  // partitions per sequence (the plan enforces it)
constexpr int kMergeParts = 8;  // partitions merged per round of loads
constexpr float kNegInf = -__builtin_huge_valf();

template <int DTYPE, int D>
struct Traits {
  static constexpr int kElemBytes = Elem<DTYPE>::bytes;
  static constexpr int kRowBytes = D * kElemBytes;     // one token row of one head
  static constexpr int kTileBytes = kTile * kRowBytes;  // 2 KiB (D=64, 16-bit) .. 8 KiB
  static constexpr int kChunk = kWaves * kTile;         // tokens per work-group iteration
  static constexpr int kLoads = kTileBytes / 1024;      // 1 KiB load instructions per tile
  static constexpr int kRowPieces = kRowBytes / 16;     // 16-byte pieces per row: 8, 16, 32
  static constexpr int kLaneElems = D / 4;              // MFMA: dims per lane per token
  static constexpr int kLanePieces = kLaneElems * kElemBytes / 16;
  static constexpr int kElemsPerPiece = 16 / kElemBytes;
  static constexpr int kWaveLds = 2 * 2 * kTileBytes;   // 2 buffers x (K, V)
  // LDS is one union, laid out per phase:
  //   tiles:  [kWaves][2 buffers][K, V][kTileBytes]
  //   merges: [0, kPartsBytes) wave o / partition (max, weight) staging,
  //           then the per-wave (max, sum) and the last-group flag.
  static constexpr int kWaveOBytes = kWaves * kMaxGroup * D * 4;     // wave merge o
  static constexpr int kPartsBytes0 = (2 * kMaxGroup * kMergeParts + 3 * kMaxGroup) * 4;  // partition merge
  static constexpr int kPartsBytes = kPartsBytes0 > kWaveOBytes ? kPartsBytes0 : kWaveOBytes;
  static constexpr int kStatsOffset = kPartsBytes;                    // s_max, s_sum
  static constexpr int kFlagOffset = kStatsOffset + 2 * kWaves * kMaxGroup * 4;
  static constexpr int kMergeEnd = kFlagOffset + 16;
  static constexpr int kLdsBytes = kWaves * kWaveLds > kMergeEnd ? kWaves * kWaveLds : kMergeEnd;
  // Work groups one CU holds (160 KiB of LDS on gfx950), and the matching
  // register budget: waves per SIMD = groups * kWaves / 4 (at least 1).
  static constexpr int kGroupsPerCU = (160 * 1024) / kLdsBytes;
  static constexpr int kWavesPerSimd = kGroupsPerCU * kWaves / 4 > 0 ? kGroupsPerCU * kWaves / 4 : 1;
  static_assert(kLoads >= 1 && kRowPieces >= 8, "tile geometry");
};

// Swizzle of the 16-byte pieces of LDS row r: slot s holds piece s ^ sw(r).
// With it, a K-operand read (16 rows, one piece each) and a transposed V
// read (rows 4g+e, two to four neighbouring pieces each) touch 16 distinct
// 4-bank groups.
template <int ROW_PIECES>
__device__ __forceinline__ int piece_swizzle(int r) {
  return ROW_PIECES == 8 ? (r >> 1) & 7 : r & 15;
}

struct DecodeArgs {
  const void* q;
  int64_t q_stride_tok, q_stride_head;  // elements
  const char* k_cache;
  const char* v_cache;
  const void* block_table;
  int64_t bt_stride;  // elements
  const int32_t* kv_len;
  const int32_t* work;  // (seq, partition, kv_len, 0) quadruples
  int32_t* counters;    // [num_seqs * num_kv_heads], zero at rest
  void* out;
  int64_t out_stride_tok, out_stride_head;  // elements
  float* ws_o;                              // [num_seqs, Hq, max_parts, D]
  float* ws_ml;                             // [num_seqs, Hq, max_parts, 2]: (max, sum)
  float scale_log2;                         // scale * log2(e)
  int32_t num_q_heads, num_kv_heads, n_rep, bs_log2, max_parts, part_tokens;
  int64_t num_blocks;
};

// --------------------------------------------------------------- MFMA ----

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

// O tile update for one 16-token tile from its swizzled LDS tile:
// o[c] += P(16 heads x 16 tokens) V(16 tokens x 16 dims), V element
// (row 4g+e, column 16c+t) per lane.
template <int DTYPE, int D>
__device__ __forceinline__ void mfma_pv(const float (&p)[4], const char* v_tile, int g, int t,
                                        f32x4 (&o)[D / 16]) {
  using Tr = Traits<DTYPE, D>;
  constexpr int RP = Tr::kRowPieces;
  constexpr int EPP = Tr::kElemsPerPiece;
  int row_base[4], row_sw[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    row_base[e] = (4 * g + e) * RP * 16;
    row_sw[e] = piece_swizzle<RP>(4 * g + e);
  }
  if constexpr (DTYPE == MV_DTYPE_F32) {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const int col = 16 * c + t;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int off = row_base[e] + (((col / EPP) ^ row_sw[e]) << 4) + (col % EPP) * 4;
        const float vv = *reinterpret_cast<const float*>(v_tile + off);
        o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[e], vv, o[c], 0, 0, 0);
      }
    }
  } else {
    s16x4 pa;
#pragma unroll
    for (int e = 0; e < 4; ++e) pa[e] = static_cast<short>(from_f32<DTYPE>(p[e]));
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const int col = 16 * c + t;
      s16x4 vb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int off = row_base[e] + (((col / EPP) ^ row_sw[e]) << 4) + (col % EPP) * 2;
        vb[e] = *reinterpret_cast<const short*>(v_tile + off);
      }
      if constexpr (DTYPE == MV_DTYPE_BF16) {
        o[c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vb, o[c], 0, 0, 0);
      } else {
        o[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, pa),
                                                    __builtin_bit_cast(f16x4, vb), o[c], 0, 0, 0);
      }
    }
  }
}

// Device-coherent (agent-scope) fp32 store / load: `global_store/load ... sc1`
// on gfx950, visible across the XCDs' separate L2 caches without any cache
// writeback or invalidate.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima): this
// wave's vector memory operations, stores included, are complete.
constexpr unsigned kWaitVmcnt0 = 0x0F70;

// Stops the compiler from moving LDS accesses of one wave across this
// point; the hardware completes one wave's LDS accesses in issue order.
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ----------------------------------------------------------- the kernel ---

// s_waitcnt vmcnt(N), N <= 63 (expcnt and lgkmcnt at their maxima; vmcnt
// is split over bits [3:0] and [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
}

template <int DTYPE, int D, typename BT>
__global__ __launch_bounds__(kWaves * 64)
__attribute__((amdgpu_waves_per_eu(Traits<DTYPE, D>::kWavesPerSimd))) void paged_decode_kernel(DecodeArgs a) {
  using Tr = Traits<DTYPE, D>;
  using raw_t = typename Elem<DTYPE>::raw;
  constexpr int L = Tr::kLoads;
  constexpr int RP = Tr::kRowPieces;
  constexpr int QP = Tr::kLanePieces;

  __shared__ __attribute__((aligned(16))) char s_lds[Tr::kLdsBytes];
  float (*s_max)[kMaxGroup] = reinterpret_cast<float (*)[kMaxGroup]>(s_lds + Tr::kStatsOffset);
  float (*s_sum)[kMaxGroup] = s_max + kWaves;
  int& s_last = *reinterpret_cast<int*>(s_lds + Tr::kFlagOffset);

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = lane & 15;  // MFMA: token row (K operand) / head column (results)
  const int g = lane >> 4;  // MFMA: dim quarter (K operand) / token quad (results)

  const int item = blockIdx.x / a.num_kv_heads;
  const int h = blockIdx.x - item * a.num_kv_heads;
  const int4 wi = reinterpret_cast<const int4*>(a.work)[item];  // (seq, partition, kv_len, -)
  const int b = wi.x;
  const int part = wi.y;
  const int kv = wi.z;
  const int n_parts = (kv + a.part_tokens - 1) / a.part_tokens;
  const int tok_begin = part * a.part_tokens;
  const int tok_end = min(kv, tok_begin + a.part_tokens);
  const int n_chunks = (tok_end - tok_begin + Tr::kChunk - 1) / Tr::kChunk;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const BT* bt_row = static_cast<const BT*>(a.block_table) + b * a.bt_stride;
  char* wave_lds = s_lds + wave * Tr::kWaveLds;  // [buffer][K, V][tile bytes]

  // LDS slot (64c + lane) of this wave's tile: its row, and the global
  // piece it holds under the swizzle.
  int slot_row[L], slot_piece[L];
#pragma unroll
  for (int c = 0; c < L; ++c) {
    const int slot = 64 * c + lane;
    slot_row[c] = slot / RP;
    slot_piece[c] = (slot % RP) ^ piece_swizzle<RP>(slot_row[c]);
  }

  // Block ids of this lane's slots in chunk `ch` (rows past the partition
  // end read the last token's entry, so every call issues L loads).
  auto load_block_ids = [&](int ch, int64_t (&blk)[L]) {
    const int tile_tok = tok_begin + ch * Tr::kChunk + wave * kTile;
#pragma unroll
    for (int c = 0; c < L; ++c) {
      const int j = min(tile_tok + slot_row[c], tok_end - 1);
      blk[c] = static_cast<int64_t>(bt_row[j >> a.bs_log2]);
    }
  };

  // Issues the HBM -> LDS loads of this wave's tile of chunk `ch` into
  // buffer `buf`; records which slots hold a token of the partition. Every
  // call issues exactly 2L load instructions (the vmcnt waits count on it):
  // slots outside the partition read the first pool row, and their V slots
  // are zeroed once the loads have landed.
  auto issue_tile = [&](int ch, int buf, const int64_t (&blk)[L], bool (&valid)[L]) {
    const int tile_tok = tok_begin + ch * Tr::kChunk + wave * kTile;
    char* kdst = wave_lds + buf * 2 * Tr::kTileBytes;
    char* vdst = kdst + Tr::kTileBytes;
#pragma unroll
    for (int c = 0; c < L; ++c) {
      const int j = tile_tok + slot_row[c];
      // the plan rejects tables with entries outside the pool; the bound
      // check only keeps a bad table from reading outside it
      const bool ok = j < tok_end && blk[c] >= 0 && blk[c] < a.num_blocks;
      const int64_t off =
          ok ? (((blk[c] * a.num_kv_heads + h) << a.bs_log2) + (j & bs_mask)) * Tr::kRowBytes +
                   slot_piece[c] * 16
             : 0;
      valid[c] = ok;
      __builtin_amdgcn_global_load_lds(a.k_cache + off, kdst + c * 1024, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(a.v_cache + off, vdst + c * 1024, 16, 0, 0);
    }
  };

  // ---- Q^T operand: head t of the group, dims of quarter g --------------
  uint4 qr[QP];
  {
    const bool ok = t < a.n_rep;
    const raw_t* qp = static_cast<const raw_t*>(a.q) + b * a.q_stride_tok +
                      (h * a.n_rep + (ok ? t : 0)) * a.q_stride_head + g * Tr::kLaneElems;
#pragma unroll
    for (int c = 0; c < QP; ++c)
      qr[c] = ok ? reinterpret_cast<const uint4*>(qp)[c] : make_uint4(0, 0, 0, 0);
  }

  float m_run = kNegInf;  // running max of head t (log2 domain)
  float l_run = 0.f;      // running sum of head t
  f32x4 o[D / 16];        // O[head 4g+e][dim 16c+t]
#pragma unroll
  for (int c = 0; c < D / 16; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Attention over this wave's tile of chunk `ch` in buffer `buf`.
  auto compute_tile = [&](int ch, int buf) {
    const char* k_tile = wave_lds + buf * 2 * Tr::kTileBytes;
    const char* v_tile = k_tile + Tr::kTileBytes;
    // S^T = K Q^T: lane (g, t) reads row t, pieces g*QP .. g*QP+QP-1
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int ksw = piece_swizzle<RP>(t);
#pragma unroll
    for (int c = 0; c < QP; ++c) {
      const uint4 kp = *reinterpret_cast<const uint4*>(k_tile + (t * RP + ((g * QP + c) ^ ksw)) * 16);
      acc = mfma_qk<DTYPE>(kp, qr[c], acc);
    }
    const int tile_tok = tok_begin + ch * Tr::kChunk + wave * kTile;
    float s[4];
    float mc = kNegInf;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[e] = tile_tok + 4 * g + e < tok_end ? acc[e] * a.scale_log2 : kNegInf;
      mc = fmaxf(mc, s[e]);
    }
    // head t's max over the tile: lanes t, t+16, t+32, t+48
    mc = fmaxf(mc, __shfl_xor(mc, 16));
    mc = fmaxf(mc, __shfl_xor(mc, 32));
    const float m_new = fmaxf(m_run, mc);
    const float m_ref = m_new == kNegInf ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_ref);
    // P = exp2(S - m), rounded to the MFMA input type; the sum uses the
    // rounded values so O / l is an exact convex combination of V rows.
    float p[4];
    float lc = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      p[e] = to_f32<DTYPE>(from_f32<DTYPE>(__builtin_amdgcn_exp2f(s[e] - m_ref)));
      lc += p[e];
    }
    lc += __shfl_xor(lc, 16);
    lc += __shfl_xor(lc, 32);
    l_run = l_run * alpha + lc;
    m_run = m_new;
    // rescale O rows (head 4g+e takes the alpha of lane 4g+e)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float ar = __shfl(alpha, 4 * g + e);
#pragma unroll
      for (int c = 0; c < D / 16; ++c) o[c][e] *= ar;
    }
    mfma_pv<DTYPE, D>(p, v_tile, g, t, o);
  };

  // Zeroes the V slots of tokens that were not loaded (P is 0 there, but
  // the stale LDS bytes could hold NaN/Inf and 0 * NaN = NaN).
  auto zero_invalid_v = [&](int buf, const bool (&valid)[L]) {
    char* vdst = wave_lds + buf * 2 * Tr::kTileBytes + Tr::kTileBytes;
#pragma unroll
    for (int c = 0; c < L; ++c)
      if (!valid[c]) *reinterpret_cast<uint4*>(vdst + c * 1024 + lane * 16) = make_uint4(0, 0, 0, 0);
  };

  // ---- tile loop ---------------------------------------------------------
  // Step ch: (1) load the block ids of chunk ch+2, (2) issue chunk ch+1's
  // tile into the other buffer, (3) wait for chunk ch's tile, (4) compute.
  // The block ids of ch+1 were loaded before chunk ch's tile was issued, so
  // using them never waits on that tile (vmcnt retires loads in order), and
  // two tiles are in flight while a third is computed.
  auto step = [&](int ch, int buf, const bool (&val_cur)[L], const int64_t (&blk_next)[L],
                  bool (&val_next)[L], int64_t (&blk_pref)[L]) {
    const bool has1 = ch + 1 < n_chunks;
    const bool has2 = ch + 2 < n_chunks;
    if (has2) load_block_ids(ch + 2, blk_pref);
    if (has1) issue_tile(ch + 1, buf ^ 1, blk_next, val_next);
    asm volatile("" ::: "memory");
    if (has2) wait_vmcnt<3 * L>();
    else if (has1) wait_vmcnt<2 * L>();
    else wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    zero_invalid_v(buf, val_cur);
    wave_lds_order();
    compute_tile(ch, buf);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the tile's LDS reads are done
    wave_lds_order();
  };
  {
    int64_t blk_a[L], blk_b[L];
    bool val_a[L], val_b[L];
    load_block_ids(0, blk_a);
    if (n_chunks > 1) load_block_ids(1, blk_b);
    issue_tile(0, 0, blk_a, val_a);
    for (int ch = 0; ch < n_chunks; ch += 2) {
      step(ch, 0, val_a, blk_b, val_b, blk_a);
      if (ch + 1 >= n_chunks) break;
      step(ch + 1, 1, val_b, blk_a, val_a, blk_b);
    }
  }

  // ---- merge the waves ------------------------------------------------------
  __syncthreads();  // every wave is done with its tiles (s_lds is reused)
  float* s_o = reinterpret_cast<float*>(s_lds);  // [kWaves][kMaxGroup][D]
  if (g == 0) {
    s_max[wave][t] = m_run;
    s_sum[wave][t] = l_run;
  }
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * g + e;  // accumulator row = query head of the group
      if (row < a.n_rep) s_o[(wave * kMaxGroup + row) * D + 16 * c + t] = o[c][e];
    }
  }
  __syncthreads();

  const int n_out = a.n_rep * D;
  const int64_t slot_base = (static_cast<int64_t>(b) * a.num_q_heads + h * a.n_rep) * a.max_parts;
  for (int idx = threadIdx.x; idx < n_out; idx += kWaves * 64) {
    const int r = idx / D;
    const int d = idx - r * D;
    float mx = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, s_max[w][r]);
    float sum = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = s_max[w][r];
      if (mw != kNegInf) {
        const float f = __builtin_amdgcn_exp2f(mw - mx);
        sum += s_sum[w][r] * f;
        acc += s_o[(w * kMaxGroup + r) * D + d] * f;
      }
    }
    if (n_parts == 1) {
      raw_t* op = static_cast<raw_t*>(a.out) + b * a.out_stride_tok + (h * a.n_rep + r) * a.out_stride_head;
      op[d] = from_f32<DTYPE>(acc / sum);
    } else {
      const int64_t slot = slot_base + static_cast<int64_t>(r) * a.max_parts + part;
      store_coherent(a.ws_o + slot * D + d, acc / sum);
      if (d == 0) {
        store_coherent(a.ws_ml + 2 * slot, mx);
        store_coherent(a.ws_ml + 2 * slot + 1, sum);
      }
    }
  }
  if (n_parts == 1) return;

  // ---- cross-partition merge by the last work group --------------------
  // The partials above are device-coherent stores; once every wave has
  // seen them acknowledged (vmcnt(0)), the counter increment publishes
  // them. The work group that completes the count reads all partials
  // with device-coherent loads. No L2 writeback/invalidate is involved.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&a.counters[b * a.num_kv_heads + h], 1,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == n_parts - 1;
  }
  __syncthreads();
  if (!s_last) return;
  // One round of loads per kMergeParts partitions: every thread issues the
  // partial values of its outputs together with its share of the
  // (max, sum) pairs, which go through LDS to form the per-head weights.
  float* s_m = reinterpret_cast<float*>(s_lds);  // [kMaxGroup][kMergeParts]
  float* s_w = s_m + kMaxGroup * kMergeParts;    // [kMaxGroup][kMergeParts]
  float* s_f = s_w + kMaxGroup * kMergeParts;    // [kMaxGroup] running max
  float* s_g = s_f + kMaxGroup;                  // [kMaxGroup] rescale of the running sums
  float* s_n = s_g + kMaxGroup;                  // [kMaxGroup] running weight sum
  constexpr int kOuts = (kMaxGroup * D + kWaves * 64 - 1) / (kWaves * 64);
  float acc[kOuts];
#pragma unroll
  for (int k = 0; k < kOuts; ++k) acc[k] = 0.f;
  if (threadIdx.x < kMaxGroup) {
    s_f[threadIdx.x] = kNegInf;
    s_n[threadIdx.x] = 0.f;
  }
  for (int p0 = 0; p0 < n_parts; p0 += kMergeParts) {
    const int np = min(kMergeParts, n_parts - p0);
    // (1) loads: partial values of this thread's outputs + (max, sum) pairs
    float ov[kOuts][kMergeParts];
#pragma unroll
    for (int k = 0; k < kOuts; ++k) {
      const int idx = threadIdx.x + k * kWaves * 64;
      const int r = idx / D;
      const int d = idx - r * D;
      const int64_t s0 = slot_base + static_cast<int64_t>(r) * a.max_parts + p0;
#pragma unroll
      for (int pp = 0; pp < kMergeParts; ++pp)
        ov[k][pp] = (idx < n_out && pp < np) ? load_coherent(a.ws_o + (s0 + pp) * D + d) : 0.f;
    }
    float mv = kNegInf, lv = 0.f;
    const int mi = threadIdx.x;  // (head, partition) pair of this thread
    const int mr = mi / kMergeParts, mp = mi - mr * kMergeParts;
    if (mi < kMaxGroup * kMergeParts && mr < a.n_rep && mp < np) {
      const int64_t sl = slot_base + static_cast<int64_t>(mr) * a.max_parts + p0 + mp;
      mv = load_coherent(a.ws_ml + 2 * sl);
      lv = load_coherent(a.ws_ml + 2 * sl + 1);
    }
    __syncthreads();  // previous round's LDS readers are done
    if (mi < kMaxGroup * kMergeParts) {
      s_m[mi] = mv;
      s_w[mi] = lv;
    }
    __syncthreads();
    // (2) per-head weights of this round, relative to the running max
    if (threadIdx.x < a.n_rep) {
      const int r = threadIdx.x;
      float mx = s_f[r];
      for (int pp = 0; pp < np; ++pp) mx = fmaxf(mx, s_m[r * kMergeParts + pp]);
      const float g = s_f[r] == kNegInf ? 0.f : __builtin_amdgcn_exp2f(s_f[r] - mx);
      float sum = s_n[r] * g;
      for (int pp = 0; pp < np; ++pp) {
        const float w = s_w[r * kMergeParts + pp] * __builtin_amdgcn_exp2f(s_m[r * kMergeParts + pp] - mx);
        s_w[r * kMergeParts + pp] = w;
        sum += w;
      }
      s_f[r] = mx;
      s_g[r] = g;
      s_n[r] = sum;
    }
    __syncthreads();
    // (3) accumulate
#pragma unroll
    for (int k = 0; k < kOuts; ++k) {
      const int idx = threadIdx.x + k * kWaves * 64;
      if (idx < n_out) {
        const int r = idx / D;
        float sacc = acc[k] * s_g[r];
#pragma unroll
        for (int pp = 0; pp < kMergeParts; ++pp) sacc += s_w[r * kMergeParts + pp] * ov[k][pp];
        acc[k] = sacc;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kOuts; ++k) {
    const int idx = threadIdx.x + k * kWaves * 64;
    if (idx < n_out) {
      const int r = idx / D;
      const int d = idx - r * D;
      raw_t* op = static_cast<raw_t*>(a.out) + b * a.out_stride_tok + (h * a.n_rep + r) * a.out_stride_head;
      op[d] = from_f32<DTYPE>(acc[k] / s_n[r]);
    }
  }
  if (threadIdx.x == 0)  // ready for the next call
    __hip_atomic_store(&a.counters[b * a.num_kv_heads + h], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------------------------- plan ---

struct PlanArgs {
  const void* kv_len;
  const void* block_table;
  int64_t bt_stride;
  int32_t num_seqs, max_blocks, bs_log2, chunk_tokens, num_kv_heads, target_groups;
  int64_t num_blocks;
  int32_t* kv_out;
  int32_t* work;
  int64_t work_cap;
  int32_t* counters;
  int32_t* status;
};

constexpr int kPlanThreads = 1024;

__device__ int block_sum(int v, int* scratch) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  int total = 0;
  for (int w = 0; w < kPlanThreads / 64; ++w) total += scratch[w];
  return total;
}

__device__ int block_max(int v, int* scratch) {
  for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  int m = 0;
  for (int w = 0; w < kPlanThreads / 64; ++w) m = max(m, scratch[w]);
  return m;
}

// One work group: validates kv_len and the table entries each sequence
// reads, picks the partition size, builds the (sequence, partition) list
// and zeroes the merge counters.
template <typename KV, typename BT>
__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(PlanArgs a) {
  __shared__ int s_scan[kPlanThreads];
  __shared__ int s_red[kPlanThreads / 64];
  __shared__ int s_cnt[4];  // bad kv_len, insufficient table, bad block id, max partitions
  __shared__ int s_min_kv;
  const int tid = threadIdx.x;
  if (tid < 4) s_cnt[tid] = 0;
  if (tid == 0) s_min_kv = INT_MAX;
  __syncthreads();

  const KV* kvp = static_cast<const KV*>(a.kv_len);
  const BT* btp = static_cast<const BT*>(a.block_table);
  const int64_t bs = int64_t(1) << a.bs_log2;
  auto valid_len = [&](int64_t kv) {
    return kv >= 1 && (kv + bs - 1) / bs <= a.max_blocks && kv <= INT_MAX / 2;
  };

  // pass 1: validate lengths, count chunks
  int chunks = 0, max_chunks = 0;
  for (int b = tid; b < a.num_seqs; b += kPlanThreads) {
    const int64_t kv = static_cast<int64_t>(kvp[b]);
    atomicMin(&s_min_kv, static_cast<int>(std::max<int64_t>(std::min<int64_t>(kv, INT_MAX), INT_MIN)));
    if (kv < 1) atomicAdd(&s_cnt[0], 1);
    else if (!valid_len(kv)) atomicAdd(&s_cnt[1], 1);
    else {
      const int c = static_cast<int>((kv + a.chunk_tokens - 1) / a.chunk_tokens);
      chunks += c;
      max_chunks = max(max_chunks, c);
    }
    a.kv_out[b] = valid_len(kv) ? static_cast<int32_t>(kv) : 0;
  }
  const int total_chunks = block_sum(chunks, s_red);
  const int most_chunks = block_max(max_chunks, s_red);
  const int64_t groups = static_cast<int64_t>(total_chunks) * a.num_kv_heads;
  // enough work groups for the device, at most kMaxParts partitions per sequence
  const int64_t target = std::max(1, a.target_groups);
  const int per_part = static_cast<int>(std::max<int64_t>(
      std::max<int64_t>(1, (groups + target - 1) / target),
      (most_chunks + kMaxParts - 1) / kMaxParts));
  const int part_tokens = per_part * a.chunk_tokens;

  // pass 2: work list
  int64_t running = 0;
  for (int base = 0; base < a.num_seqs; base += kPlanThreads) {
    const int b = base + tid;
    int np = 0;
    if (b < a.num_seqs) {
      const int64_t kv = static_cast<int64_t>(kvp[b]);
      if (valid_len(kv)) {
        np = static_cast<int>((kv + part_tokens - 1) / part_tokens);
        atomicMax(&s_cnt[3], np);
      }
    }
    s_scan[tid] = np;
    __syncthreads();
    for (int off = 1; off < kPlanThreads; off <<= 1) {
      const int v = tid >= off ? s_scan[tid - off] : 0;
      __syncthreads();
      s_scan[tid] += v;
      __syncthreads();
    }
    const int64_t start = running + s_scan[tid] - np;
    for (int p = 0; p < np; ++p) {
      const int64_t idx = start + p;
      if (idx < a.work_cap) {
        reinterpret_cast<int4*>(a.work)[idx] = make_int4(b, p, static_cast<int>(kvp[b]), 0);
      }
    }
    running += s_scan[kPlanThreads - 1];
    __syncthreads();
  }

  // pass 3: every table entry a valid sequence reads must be a pool block
  const int64_t n = static_cast<int64_t>(a.num_seqs) * a.max_blocks;
  int bad = 0;
  for (int64_t i = tid; i < n; i += kPlanThreads) {
    const int64_t b = i / a.max_blocks;
    const int64_t j = i - b * a.max_blocks;
    const int64_t kv = static_cast<int64_t>(kvp[b]);
    if (!valid_len(kv)) continue;
    if (j < (kv + bs - 1) / bs) {
      const int64_t blk = static_cast<int64_t>(btp[b * a.bt_stride + j]);
      bad += (blk < 0 || blk >= a.num_blocks);
    }
  }
  if (bad) atomicAdd(&s_cnt[2], bad);
  const int64_t nc = static_cast<int64_t>(a.num_seqs) * a.num_kv_heads;
  for (int64_t i = tid; i < nc; i += kPlanThreads) a.counters[i] = 0;
  __syncthreads();
  if (tid == 0) {
    a.status[MV_PLAN_NUM_ITEMS] = static_cast<int32_t>(std::min<int64_t>(running, INT_MAX));
    a.status[MV_PLAN_BAD_KV_LEN] = s_cnt[0];
    a.status[MV_PLAN_INSUFFICIENT] = s_cnt[1];
    a.status[MV_PLAN_BAD_BLOCK] = s_cnt[2];
    a.status[MV_PLAN_MAX_PARTS] = s_cnt[3];
    a.status[MV_PLAN_MIN_KV_LEN] = a.num_seqs > 0 ? s_min_kv : 0;
    a.status[MV_PLAN_PARTITION_TOKENS] = part_tokens;
    a.status[7] = 0;
  }
}

// ------------------------------------------------------------- dispatch ---

size_t ws_o_bytes(int64_t num_seqs, int64_t hq, int64_t d, int64_t parts) {
  return static_cast<size_t>(num_seqs * hq * parts * d * 4);
}

template <template <int, int> class Q>
int trait_value(int head_dim, int dtype) {
  const bool d64 = head_dim == 64;
  switch (dtype) {
    case MV_DTYPE_F32: return d64 ? Q<MV_DTYPE_F32, 64>::value : Q<MV_DTYPE_F32, 128>::value;
    case MV_DTYPE_F16: return d64 ? Q<MV_DTYPE_F16, 64>::value : Q<MV_DTYPE_F16, 128>::value;
    default: return d64 ? Q<MV_DTYPE_BF16, 64>::value : Q<MV_DTYPE_BF16, 128>::value;
  }
}
template <int DTYPE, int D> struct ChunkOf { static constexpr int value = Traits<DTYPE, D>::kChunk; };
template <int DTYPE, int D> struct GroupsOf { static constexpr int value = Traits<DTYPE, D>::kGroupsPerCU; };

int chunk_tokens(int head_dim, int dtype) { return trait_value<ChunkOf>(head_dim, dtype); }

template <int DTYPE, int D, typename BT>
int launch_decode(const DecodeArgs& a, int num_items, hipStream_t s) {
  const int64_t grid = static_cast<int64_t>(num_items) * a.num_kv_heads;
  if (grid > INT_MAX) return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: grid too large");
  paged_decode_kernel<DTYPE, D, BT><<<static_cast<unsigned>(grid), kWaves * 64, 0, s>>>(a);
  return check_launch("mv_paged_decode");
}

template <int DTYPE, int D>
int launch_decode_bt(const DecodeArgs& a, bool bt64, int num_items, hipStream_t s) {
  return bt64 ? launch_decode<DTYPE, D, int64_t>(a, num_items, s)
              : launch_decode<DTYPE, D, int32_t>(a, num_items, s);
}

template <int DTYPE>
int launch_decode_d(const DecodeArgs& a, int d, bool bt64, int num_items, hipStream_t s) {
  return d == 64 ? launch_decode_bt<DTYPE, 64>(a, bt64, num_items, s)
                 : launch_decode_bt<DTYPE, 128>(a, bt64, num_items, s);
}

}  // namespace
}  // namespace mv

extern "C" int mv_decode_chunk_tokens(int32_t head_dim, int32_t dtype) {
  if ((head_dim != 64 && head_dim != 128) || mv::dtype_bytes(dtype) == 0) return 0;
  return mv::chunk_tokens(head_dim, dtype);
}

extern "C" int mv_decode_groups_per_cu(int32_t head_dim, int32_t dtype) {
  if ((head_dim != 64 && head_dim != 128) || mv::dtype_bytes(dtype) == 0) return 0;
  return mv::trait_value<mv::GroupsOf>(head_dim, dtype);
}

extern "C" size_t mv_paged_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                  int32_t head_dim, int32_t max_partitions) {
  if (max_partitions <= 1 || num_seqs <= 0 || num_q_heads <= 0 || head_dim <= 0) return 0;
  const size_t o = mv::ws_o_bytes(num_seqs, num_q_heads, head_dim, max_partitions);
  const size_t ml = static_cast<size_t>(num_seqs) * num_q_heads * max_partitions * sizeof(float2);
  return ((o + 255) / 256) * 256 + ml;
}

extern "C" int mv_decode_plan(const void* kv_len, int32_t kv_len_is_i64, const void* block_table,
                              int32_t bt_is_i64, int64_t bt_stride, int32_t num_seqs,
                              int32_t max_blocks, int32_t block_size, int64_t num_blocks,
                              int32_t chunk_tokens, int32_t num_kv_heads, int32_t target_groups,
                              int32_t* kv_len_i32, int32_t* work_items, int64_t work_capacity,
                              int32_t* counters, int32_t* status, void* stream) {
  using namespace mv;
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_plan: null status");
  if (num_seqs < 0 || max_blocks < 0 || work_capacity < 0 || num_blocks < 0 || num_kv_heads <= 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_plan: bad sizes");
  if (chunk_tokens <= 0 || chunk_tokens % kTile)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_plan: chunk_tokens %d", chunk_tokens);
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "mv_decode_plan: block_size %d is not a power of 2", block_size);
  if (num_seqs > 0 && (!kv_len || !kv_len_i32 || !counters || (max_blocks > 0 && !block_table)))
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_plan: null pointer");
  if (work_capacity > 0 && !work_items)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_plan: null work list");
  PlanArgs a;
  a.kv_len = kv_len;
  a.block_table = block_table;
  a.bt_stride = bt_stride;
  a.num_seqs = num_seqs;
  a.max_blocks = max_blocks;
  a.bs_log2 = ilog2_exact(block_size);
  a.chunk_tokens = chunk_tokens;
  a.num_kv_heads = num_kv_heads;
  a.target_groups = target_groups;
  a.num_blocks = num_blocks;
  a.kv_out = kv_len_i32;
  a.work = work_items;
  a.work_cap = work_capacity;
  a.counters = counters;
  a.status = status;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (kv_len_is_i64) {
    if (bt_is_i64) decode_plan_kernel<int64_t, int64_t><<<1, kPlanThreads, 0, s>>>(a);
    else decode_plan_kernel<int64_t, int32_t><<<1, kPlanThreads, 0, s>>>(a);
  } else {
    if (bt_is_i64) decode_plan_kernel<int32_t, int64_t><<<1, kPlanThreads, 0, s>>>(a);
    else decode_plan_kernel<int32_t, int32_t><<<1, kPlanThreads, 0, s>>>(a);
  }
  return check_launch("mv_decode_plan");
}

extern "C" int mv_paged_decode(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                               const void* key_cache, const void* value_cache,
                               const void* block_table, int32_t bt_is_i64, int64_t bt_stride,
                               const int32_t* kv_len_i32, const int32_t* work_items,
                               int32_t num_work_items, int32_t partition_tokens,
                               int32_t max_partitions, int32_t* counters, void* out,
                               int64_t out_stride_tok, int64_t out_stride_head, float scale,
                               int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                               int32_t head_dim, int32_t block_size, int64_t num_blocks,
                               int32_t dtype, void* workspace, size_t workspace_bytes,
                               void* stream) {
  using namespace mv;
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(MV_ERR_UNSUPPORTED, "mv_paged_decode: unknown dtype %d", dtype);
  if (head_dim != 64 && head_dim != 128)
    return fail(MV_ERR_UNSUPPORTED, "mv_paged_decode: head_dim %d not supported (64, 128)", head_dim);
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "mv_paged_decode: block_size %d is not a power of 2", block_size);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_paged_decode: num_q_heads %d not divisible by num_kv_heads %d", num_q_heads,
                num_kv_heads);
  const int n_rep = num_q_heads / num_kv_heads;
  if (n_rep > kMaxGroup)
    return fail(MV_ERR_UNSUPPORTED, "mv_paged_decode: %d query heads per kv head (max %d)", n_rep,
                kMaxGroup);
  if (num_seqs < 0 || num_work_items < 0 || num_blocks <= 0 || max_partitions < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: bad sizes");
  const int chunk = chunk_tokens(head_dim, dtype);
  if (partition_tokens <= 0 || partition_tokens % chunk)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_paged_decode: partition_tokens %d is not a positive multiple of %d",
                partition_tokens, chunk);
  if (num_seqs == 0 || num_work_items == 0) return MV_OK;
  if (!query || !key_cache || !value_cache || !block_table || !kv_len_i32 || !work_items || !out)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: null pointer");
  // 16-byte loads of q rows and cache rows.
  if ((reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(key_cache) |
       reinterpret_cast<uintptr_t>(value_cache)) % 16 ||
      (q_stride_tok * eb) % 16 || (q_stride_head * eb) % 16)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: query/cache rows not 16-byte aligned");
  if (max_partitions > 0 && num_work_items > max_partitions * static_cast<int64_t>(num_seqs))
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: work list larger than the plan allows");

  DecodeArgs a;
  a.q = query;
  a.q_stride_tok = q_stride_tok;
  a.q_stride_head = q_stride_head;
  a.k_cache = static_cast<const char*>(key_cache);
  a.v_cache = static_cast<const char*>(value_cache);
  a.block_table = block_table;
  a.bt_stride = bt_stride;
  a.kv_len = kv_len_i32;
  a.work = work_items;
  a.counters = counters;
  a.out = out;
  a.out_stride_tok = out_stride_tok;
  a.out_stride_head = out_stride_head;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.n_rep = n_rep;
  a.bs_log2 = ilog2_exact(block_size);
  a.max_parts = max_partitions;
  a.part_tokens = partition_tokens;
  a.num_blocks = num_blocks;
  a.ws_o = nullptr;
  a.ws_ml = nullptr;
  if (max_partitions > 1) {
    const size_t need =
        mv_paged_decode_workspace_bytes(num_seqs, num_q_heads, head_dim, max_partitions);
    if (!workspace || workspace_bytes < need)
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: workspace %zu bytes, need %zu",
                  workspace_bytes, need);
    if (reinterpret_cast<uintptr_t>(workspace) % 256)
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: workspace not 256-byte aligned");
    if (!counters) return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: null counters");
    const size_t o = ws_o_bytes(num_seqs, num_q_heads, head_dim, max_partitions);
    a.ws_o = static_cast<float*>(workspace);
    a.ws_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((o + 255) / 256) * 256);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bt64 = bt_is_i64 != 0;
  switch (dtype) {
    case MV_DTYPE_F32: return launch_decode_d<MV_DTYPE_F32>(a, head_dim, bt64, num_work_items, s);
    case MV_DTYPE_F16: return launch_decode_d<MV_DTYPE_F16>(a, head_dim, bt64, num_work_items, s);
    default: return launch_decode_d<MV_DTYPE_BF16>(a, head_dim, bt64, num_work_items, s);
  }
}
