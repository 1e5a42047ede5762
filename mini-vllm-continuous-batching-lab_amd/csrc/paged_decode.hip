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
// Prologue (one dependent memory round trip before the first tile):
//   the work item (seq, partition, kv_len) and the partition's pool block
//   ids, both addressed by blockIdx alone (the plan kernel stores each
//   item's ids), arrive together; the ids go straight to LDS. The group's
//   Q rows are then copied to LDS alongside the first tiles.
//
// Per tile (16 tokens x D) and wave, with lane = 16*g + t (g = 0..3):
//   * HBM -> LDS without registers: global_load_lds_dwordx4 (non-temporal:
//     each K/V byte is read once) writes lane l's
//     16 bytes to LDS slot (64c + l) of load instruction c. Each lane
//     fetches the 16-byte piece that belongs in its slot under an XOR
//     swizzle (slot s of row r holds piece s ^ sw(r)), so every load
//     instruction still reads 1 KiB of contiguous HBM while the reads
//     below are bank-conflict free with unpadded rows. kStages buffers per
//     wave: up to kStages - 1 tiles stream in while one is computed, with
//     exact vmcnt waits (the copies are issued through inline asm so the
//     compiler does not drain them before every LDS access).
//   * S^T = K Q^T on MFMA (16x16x32 for 16-bit types, 16x16x4 for fp32):
//     A = K tile (M = tokens), row t, dims [g*D/4, (g+1)*D/4) from LDS;
//     B = Q^T (N = query heads of the group; columns >= n_rep repeat a
//     real head and are never stored) from registers. Both operands use
//     the same k-slot -> dim mapping, so the contraction covers all D dims
//     whatever the hardware's k order.
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
// reduce (device-coherent loads, one round of loads per up to 16
// partitions), writes the output and resets the counter to zero. (A
// __threadfence() here would write back and invalidate the whole L2 of the
// XCD in every wave, which costs ~10x the kernel.) Counters are zeroed by
// the plan kernel, so every call that shares a plan must run on one stream.
#include <algorithm>
#include <atomic>
#include <climits>
#include <mutex>

#include "mv_coherent.h"
#include "mv_common.h"
#include "mv_rope.h"
#include "mv_step_check.h"
#include "mv_tile.h"

namespace mv {
namespace {

// Launch geometry (build-time tunables; the defaults are the shipped shape).
#ifndef MV_DECODE_WAVES
#define MV_DECODE_WAVES 4
#endif
#ifndef MV_DECODE_STAGES
#define MV_DECODE_STAGES 2
#endif
constexpr int kWaves = MV_DECODE_WAVES;
constexpr int kMaxParts = 128;  // partitions per sequence the plan aims for
constexpr int kIdCap = 512;     // block ids one partition may span (staged in LDS)
constexpr int kIdsFirst = 64;   // ids copied before the work item is known, for long id lists
constexpr int kFewUnitsPerCU = 2;   // plan target when the (sequence, kv head) units fit the CUs
constexpr int kManyUnitsPerCU = 3;  // plan target cap otherwise

template <int DTYPE, int D, int SREQ = MV_DECODE_STAGES>
struct Traits : TileGeom<DTYPE, D> {
  using G = TileGeom<DTYPE, D>;
  using G::kElemBytes;
  using G::kRowBytes;
  using G::kTileBytes;
  using G::kLoads;
  using G::kRowPieces;
  using G::kLaneElems;
  using G::kLanePieces;
  using G::kElemsPerPiece;
  static constexpr int kChunk = kWaves * kTile;         // tokens per work-group iteration
  // Tile buffers per wave: up to S-1 tiles stream in while one is computed.
  // Larger tiles get at most 2 stages so two work groups still fit one CU.
  // SREQ = 2 by default; 3 for launches of short pieces over few units
  // (kDeepPieceTokens): see launch_decode.
  static constexpr int kStages = kTileBytes <= 2048 ? SREQ : (SREQ < 2 ? SREQ : 2);
  static constexpr int kStageBytes = 2 * kTileBytes;    // K tile, V tile
  static constexpr int kWaveLds = kStages * kStageBytes;
  // LDS is one union, laid out per phase:
  //   tile loop: [kWaves][kStages][K, V][kTileBytes], then the partition's
  //              block ids (int32, kIdCap), then the group's 16 Q rows, then
  //              the cos and sin rows of the sequence's position (fused RoPE),
  //              the new K and V rows and the new token's slot (fused write);
  //   epilogue:  each wave's o rows and (max, sum) in its own tile buffers;
  //              the last-group flag where the block ids were.
  static constexpr int kIdsOffset = kWaves * kWaveLds;
  static constexpr int kQOffset = kIdsOffset + kIdCap * 4;  // Q rows of the group (16 x D)
  static constexpr int kQLoads = kTile * kRowBytes / 1024;  // 1 KiB copies of the Q rows
  static constexpr int kTilesEnd = kQOffset + kTile * kRowBytes;
  // Wave merge o rows, padded by 4 floats: the accumulator rows 4g+e that
  // one store instruction writes then start 16 banks apart.
  static constexpr int kORowStride = D + 4;
  static constexpr int kWaveEpilogueBytes = (kMaxGroup * kORowStride + 2 * kMaxGroup) * 4;
  static constexpr int kFlagOffset = kIdsOffset;
  static constexpr int kRopeOffset = kTilesEnd;  // cos row, then sin row (kRowBytes each)
  static constexpr int kNewOffset = kRopeOffset + 2 * kRowBytes;  // new K row, then V row (fused write)
  static constexpr int kSlotOffset = kNewOffset + 2 * kRowBytes;  // the new token's slot (int64)
  static constexpr int kLdsBytes = kSlotOffset + 16;
  static_assert(kWaveEpilogueBytes <= kWaveLds, "a wave's epilogue fits its tile buffers");
  static_assert(kStages >= 2 && kStages <= 4, "tile stages");
  // Work groups one CU holds (160 KiB of LDS on gfx950), and the matching
  // register budget: waves per SIMD = groups * kWaves / 4 (at least 1).
  static constexpr int kGroupsPerCU = (160 * 1024) / kLdsBytes;
  static constexpr int kWavesPerSimd = kGroupsPerCU * kWaves / 4 > 0 ? kGroupsPerCU * kWaves / 4 : 1;
  // Epilogue: 16 threads per query head, D/32 dim pairs each; the
  // partition merge folds up to kMergeRound partitions per round of loads.
  static constexpr int kPairsPerThread = D / 32;
  static constexpr int kMergeRound = 1024 / D;
  static_assert(kLoads >= 1 && kRowPieces >= 8, "tile geometry");
  static_assert(kWaves * 64 >= 256 || kWaves * 64 % 16 == 0, "epilogue mapping");
};

// Kernel arguments; the fields the prologue needs come first, so a couple
// of wide scalar loads fetch them together.
struct DecodeArgs {
  const int32_t* work;       // per work group: (seq, kv head, piece, pieces, token begin, end, 0, 0)
  const int32_t* block_ids;  // [work group][ids_per_item]: the piece's pool blocks first
  const void* q;
  const char* k_cache;
  const char* v_cache;
  int64_t q_stride_tok, q_stride_head;  // elements
  int32_t ids_per_item;                 // multiple of 4, <= kIdCap
  int32_t num_kv_heads, n_rep, bs_log2;
  float scale_log2;                     // scale * log2(e)
  int32_t num_q_heads, max_parts;
  uint32_t num_blocks_u32;  // pool blocks (at most 2^31): ids at or above are not read
  float inv_scale_log2;  // 1 / scale_log2
  int32_t* counters;  // [num_seqs * num_kv_heads], zero at rest
  void* out;
  int64_t out_stride_tok, out_stride_head;  // elements
  float* ws_o;                              // [num_seqs, Hq, max_parts, D], 16-bit rows for F16/BF16
  float* ws_ml;                             // [num_seqs, Hq, max_parts, 2]: (max, sum)
  // Fused KV write of the step's new tokens (FUSED kernels only): row b of
  // new_k / new_v goes to pool slot slots[b].
  const char* new_k;
  const char* new_v;
  int64_t nk_st, nk_sh, nv_st, nv_sh;  // bytes
  const int64_t* slots;
  int64_t total_slots;
  // Fused RoPE of the query and the new key (FUSED kernels, optional): the
  // cos / sin table rows at each sequence's position, [num_seqs][D].
  const char* rope_cos;
  const char* rope_sin;
};

// --------------------------------------------------------------- MFMA ----

// Split-K partial O rows of 16-bit data in the data's own type: a partial
// row is a convex combination of V rows, so the type holds it, and the
// final output is rounded to that type anyway. Half the bytes of fp32
// partials on the merge's critical tail (stores, then the merger's loads);
// the (max, sum) pairs stay fp32.
#ifndef MV_DECODE_PARTIALS16
#define MV_DECODE_PARTIALS16 1
#endif
#ifndef MV_DECODE_EARLY_V
#define MV_DECODE_EARLY_V 1
#endif

// A tile keeps p = exp2(s - m) with the head's reference m unchanged when
// every head's tile sum lies in [kLazyMin, kLazyMax].
constexpr float kLazyMax = 4096.f;
constexpr float kLazyMin = 1.f / 4096.f;

// ----------------------------------------------------------- the kernel ---

template <int DTYPE, int D, bool FUSED, bool ROPE, int SREQ = MV_DECODE_STAGES>
__global__ __launch_bounds__(kWaves * 64)
__attribute__((amdgpu_waves_per_eu(Traits<DTYPE, D, SREQ>::kWavesPerSimd))) void paged_decode_kernel(DecodeArgs a) {
  static_assert(FUSED || !ROPE, "the fused RoPE comes with the fused write");
  constexpr bool kPartials16 = DTYPE != MV_DTYPE_F32 && MV_DECODE_PARTIALS16;
  using Tr = Traits<DTYPE, D, SREQ>;
  using raw_t = typename Elem<DTYPE>::raw;
  constexpr int L = Tr::kLoads;
  constexpr int RP = Tr::kRowPieces;
  constexpr int QP = Tr::kLanePieces;

  __shared__ __attribute__((aligned(16))) char s_lds[Tr::kLdsBytes];
  int& s_last = *reinterpret_cast<int*>(s_lds + Tr::kFlagOffset);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int t = lane & 15;  // MFMA: token row (K operand) / head column (results)
  const int g = lane >> 4;  // MFMA: dim quarter (K operand) / token quad (results)

  // The kernel arguments the prologue needs, in SGPRs at once: otherwise
  // the compiler loads them field by field with a wait in between, which
  // costs several scalar memory round trips before the first copy.
  asm volatile("" ::"s"(a.work), "s"(a.block_ids), "s"(a.ids_per_item), "s"(a.num_kv_heads),
               "s"(a.q), "s"(a.q_stride_tok), "s"(a.q_stride_head), "s"(a.n_rep), "s"(a.k_cache),
               "s"(a.v_cache), "s"(a.bs_log2));
  if constexpr (FUSED)  // the new rows' and the slot's copies, before the tile loop
    asm volatile("" ::"s"(a.new_k), "s"(a.new_v), "s"(a.nk_st), "s"(a.nk_sh), "s"(a.nv_st), "s"(a.nv_sh),
                 "s"(a.slots));
  if constexpr (ROPE) asm volatile("" ::"s"(a.rope_cos), "s"(a.rope_sin));
  const int item = blockIdx.x;
  const uint32_t lds0 = lds_address(s_lds);
  int32_t* s_ids = reinterpret_cast<int32_t*>(s_lds + Tr::kIdsOffset);

  // ---- the work item and its block ids: both addressed by blockIdx alone,
  // so they travel together (one memory round trip). Wave 0 copies the
  // first window of the list: all of it when the list is at most 256 ids
  // (a plan sized for this step's pieces), else kIdsFirst ids (a launch of
  // fixed size, whose lists have the widest piece's stride: most pieces
  // need far fewer, and unused slots none). Lanes past the window re-read
  // its last 16 bytes. The copy is issued first: the work item's scalar
  // load must not sit in front of it (a wait for it would also cover the
  // kernel arguments the copy needs).
  const int first_ids = a.ids_per_item <= 256 ? a.ids_per_item : kIdsFirst;
  const int64_t ids_base = static_cast<int64_t>(item) * a.ids_per_item;
  if (wave == 0) {
    const int32_t* src = a.block_ids + ids_base + min(4 * lane, first_ids - 4);
    copy_to_lds_16B(reinterpret_cast<const char*>(src), __builtin_amdgcn_readfirstlane(lds0 + Tr::kIdsOffset));
  }
  asm volatile("" ::: "memory");
  const int4 w0 = reinterpret_cast<const int4*>(a.work + 8 * static_cast<int64_t>(item))[0];
  const int4 w1 = reinterpret_cast<const int4*>(a.work + 8 * static_cast<int64_t>(item))[1];
  wait_vmcnt<0>();
  asm volatile("" ::: "memory");
  if (w0.x < 0) return;      // an unused slot of a fixed-size launch (no copy in flight)
  const int b = w0.x;        // sequence
  const int h = w0.y;        // kv head
  const int part = w0.z;     // piece of the sequence
  const int n_parts = w0.w;  // pieces of the sequence
  const int tok_begin = w1.x;
  const int tok_end = w1.y;
  const int n_chunks = (tok_end - tok_begin + Tr::kChunk - 1) / Tr::kChunk;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const int first_blk = tok_begin >> a.bs_log2;  // s_ids[i] = pool block of table entry first_blk + i
  {
    // All the ids when the piece spans more table entries than the first
    // window held (a second round trip, for long pieces only): wave w
    // copies ids [256 w, 256 w + 256) of [0, need) to their LDS slots (the
    // first window again, with the same values); lanes past `need` re-read
    // its last 16 bytes, so no copy leaves the item's list or the LDS id
    // buffer (kWaves * 256 >= kIdCap).
    static_assert(kWaves * 256 >= kIdCap, "the id copy covers the id buffer");
    const int need = min((((tok_end - 1) >> a.bs_log2) - first_blk + 1 + 3) & ~3, a.ids_per_item);
    if (need > first_ids) {
      if (wave * 256 < need) {
        const int32_t* src = a.block_ids + ids_base + min(wave * 256 + 4 * lane, need - 4);
        copy_to_lds_16B(reinterpret_cast<const char*>(src),
                        __builtin_amdgcn_readfirstlane(lds0 + Tr::kIdsOffset + wave * 1024));
      }
      wait_vmcnt<0>();
      asm volatile("" ::: "memory");
    }
  }
  const char* wave_tiles = s_lds + wave * Tr::kWaveLds;  // [stage][K, V][tile bytes]
  const uint32_t wave_tiles_lds = lds0 + wave * Tr::kWaveLds;

  // ---- fused KV write (FUSED): the work group holding sequence b's last
  // token stores the new K / V rows of b into slot slots[b] before its tile
  // loop. When that slot is the token's table position (as the block
  // manager lays it out) the token's row in the LDS tile is overwritten
  // with the new rows -- the bytes the write stores -- before it is used;
  // otherwise the token is the one read from the pool. The rows and the
  // slot arrive in LDS with the Q rows (wave 0's copies, before any tile
  // copy); wave new_wave (the one whose tile holds the token) then keeps
  // the rows in registers, lanes [0, RP) the K row's 16-byte pieces,
  // [RP, 2 RP) the V row's, and with the fused RoPE rotates the K row
  // there, before its tile loop: off the tail of the sequence's last piece
  // (0.6 us per layer call when it was done at the last tile). The tile
  // copies themselves are those of the plain kernel.
  const bool last_piece = FUSED && part == n_parts - 1;
  const int new_wave = ((tok_end - 1 - tok_begin) / kTile) % kWaves;
  int64_t new_slot = -1;
  uint4 new_piece = make_uint4(0, 0, 0, 0);
  const bool new_lane = wave == new_wave && lane < 2 * RP;
  const int new_pc = lane < RP ? lane : lane - RP;

  // ---- Q rows of the group -> LDS (wave 0). Rows r >= n_rep repeat row
  // n_rep - 1: MFMA columns (and the softmax state per column) are
  // independent, and those columns are never written out.
  if (wave == 0) {
#pragma unroll
    for (int c = 0; c < Tr::kQLoads; ++c) {
      const int byte = c * 1024 + 16 * lane;
      const int row = byte / Tr::kRowBytes;
      const int col = (byte % Tr::kRowBytes) / Tr::kElemBytes;
      const raw_t* src = static_cast<const raw_t*>(a.q) + b * a.q_stride_tok +
                         (h * a.n_rep + min(row, a.n_rep - 1)) * a.q_stride_head + col;
      copy_to_lds_16B(reinterpret_cast<const char*>(src),
                      __builtin_amdgcn_readfirstlane(lds0 + Tr::kQOffset + c * 1024));
    }
    // the sequence's cos and sin rows (fused RoPE): lanes [0, RP) the cos
    // row's 16-byte pieces, [RP, 2 RP) the sin row's, to the LDS rows after Q
    if (ROPE && lane < 2 * RP) {
      const char* src = (lane < RP ? a.rope_cos : a.rope_sin) + static_cast<int64_t>(b) * Tr::kRowBytes +
                        (lane < RP ? lane : lane - RP) * 16;
      copy_to_lds_16B(src, __builtin_amdgcn_readfirstlane(lds0 + Tr::kRopeOffset));
    }
    // the sequence's new K and V rows (fused write, last piece): lanes
    // [0, RP) the K row's pieces, [RP, 2 RP) the V row's, to the LDS rows
    // after the cos and sin rows
    if (FUSED && last_piece && lane < 2 * RP) {
      const char* src = (lane < RP ? a.new_k + b * a.nk_st + h * a.nk_sh : a.new_v + b * a.nv_st + h * a.nv_sh) +
                        new_pc * 16;
      copy_to_lds_16B(src, __builtin_amdgcn_readfirstlane(lds0 + Tr::kNewOffset));
    }
    // and the slot of b's new token: lanes 0 and 1 copy its two 32-bit
    // halves (a register load here would be waited for at once, one more
    // memory round trip before this group's first tile)
    if (FUSED && last_piece && lane < 2)
      copy_to_lds_4B(reinterpret_cast<const char*>(a.slots + b) + 4 * lane,
                     __builtin_amdgcn_readfirstlane(lds0 + Tr::kSlotOffset));
  }

  // LDS slot (64c + lane) of this wave's tile: its row, and the global
  // piece it holds under the swizzle.
  int slot_row[L], slot_piece[L];
#pragma unroll
  for (int c = 0; c < L; ++c) {
    const int slot = 64 * c + lane;
    slot_row[c] = slot / RP;
    slot_piece[c] = (slot % RP) ^ piece_swizzle<RP>(slot_row[c]);
  }
  __syncthreads();  // block ids visible to every wave

  // Issues the HBM -> LDS copies of this wave's tile of chunk `k` into
  // stage ST and returns, one bit per load, which slots hold a token of the
  // partition. Every call issues exactly 2L load instructions (the vmcnt
  // waits count on it): slots outside the partition read the first pool
  // row, and their V slots are zeroed once the loads have landed.
  auto issue_tile = [&](int k, auto st_c) __attribute__((always_inline)) -> unsigned {
    constexpr int ST = decltype(st_c)::value;
    const int tile_tok = tok_begin + k * Tr::kChunk + wave * kTile;
    const uint32_t kdst = wave_tiles_lds + ST * Tr::kStageBytes;
    // A whole tile in one pool block (block size >= 16; pieces start on
    // tile boundaries): one wave-uniform base in SGPRs and a 32-bit offset
    // per lane, no per-lane 64-bit address arithmetic.
    if (a.bs_log2 >= 4 && tile_tok + kTile <= tok_end) {
      const int id = __builtin_amdgcn_readfirstlane(s_ids[min((tile_tok >> a.bs_log2) - first_blk, kIdCap - 1)]);
      const bool ok = static_cast<uint32_t>(id) < a.num_blocks_u32;  // -1 and stale ids fail
      const int64_t row0 = ok ? ((static_cast<int64_t>(id) * a.num_kv_heads + h) << a.bs_log2) + (tile_tok & bs_mask) : 0;
      const char* bk = a.k_cache + row0 * Tr::kRowBytes;
      const char* bv = a.v_cache + row0 * Tr::kRowBytes;
#pragma unroll
      for (int c = 0; c < L; ++c) {
        const uint32_t lane_off = static_cast<uint32_t>(slot_row[c] * Tr::kRowBytes + slot_piece[c] * 16);
        copy_to_lds_16B_sv_stream(bk, lane_off, __builtin_amdgcn_readfirstlane(kdst + c * 1024));
        copy_to_lds_16B_sv_stream(bv, lane_off, __builtin_amdgcn_readfirstlane(kdst + Tr::kTileBytes + c * 1024));
      }
      return ok ? (1u << L) - 1 : 0u;
    }
    int64_t off[L];
    unsigned valid = 0;
#pragma unroll
    for (int c = 0; c < L; ++c) {
      const int j = tile_tok + slot_row[c];
      const int jj = min(j, tok_end - 1);
      const int id = s_ids[min((jj >> a.bs_log2) - first_blk, kIdCap - 1)];  // -1: not a pool block
      const bool ok = j < tok_end && static_cast<uint32_t>(id) < a.num_blocks_u32;  // -1 and stale ids fail
      off[c] = ok ? (((static_cast<int64_t>(id) * a.num_kv_heads + h) << a.bs_log2) + (jj & bs_mask)) *
                            Tr::kRowBytes +
                        slot_piece[c] * 16
                  : 0;
      valid |= ok ? (1u << c) : 0u;
    }
#pragma unroll
    for (int c = 0; c < L; ++c) {
      copy_to_lds_16B_stream(a.k_cache + off[c], __builtin_amdgcn_readfirstlane(kdst + c * 1024));
      copy_to_lds_16B_stream(a.v_cache + off[c],
                      __builtin_amdgcn_readfirstlane(kdst + Tr::kTileBytes + c * 1024));
    }
    return valid;
  };

  uint4 qr[QP];  // Q^T operand: head t of the group, dims of quarter g (from LDS)
  // head t's reference m (log2 domain; not necessarily its running max)
  // and running sum, with O and l relative to m
  float m_run = 0.f;
  float l_run = 0.f;
  f32x4 o[D / 16];        // O[head 4g+e][dim 16c+t]
#pragma unroll
  for (int c = 0; c < D / 16; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Attention over this wave's tile of chunk `k` in stage `st`.
  auto compute_tile = [&](int k, int st) __attribute__((always_inline)) {
    const char* k_tile = wave_tiles + st * Tr::kStageBytes;
    const char* v_tile = k_tile + Tr::kTileBytes;
    // 16-bit types: the P V operands are read from LDS with the K operands,
    // at the start of the tile (MV_DECODE_EARLY_V), not after the softmax:
    // the PV MFMAs then wait for no LDS round trip of their own
    constexpr bool kEarlyV = DTYPE != MV_DTYPE_F32 && MV_DECODE_EARLY_V;
    s16x4 vb[D / 16];
    if constexpr (kEarlyV) read_v_operands<DTYPE, D>(v_tile, g, t, vb);
    // the MFMAs start from -m / (scale log2 e): acc * scale log2 e = s - m
    const float c0 = -m_run * a.inv_scale_log2;
    f32x4 acc = {c0, c0, c0, c0};
#if defined(MV_DECODE_QK_VALU)
    if constexpr (!ROPE) {
      // Build-time alternative for measurement (MFMA against VALU): S^T by
      // VALU dot products, lane (g, t) computing tokens 4g..4g+3 of head t
      // over all D dims, Q row t read from LDS, K rows through the swizzle.
      // Lane t starts at piece t mod RP: the 16 Q rows sit 128 bytes apart,
      // so reading one piece of every row at once hits the same banks (8-way
      // at D = 64). Unrolled by 4 pieces: a full unroll hoists every LDS
      // read of the tile ahead of the dot products and spills (468 B/lane at
      // bf16 D=64), and so does holding the Q row in registers.
      const char* q_row = s_lds + Tr::kQOffset + t * Tr::kRowBytes;
#pragma unroll 4
      for (int pi = 0; pi < RP; ++pi) {
        const int pc = (pi + t) & (RP - 1);
        const uint4 qv = *reinterpret_cast<const uint4*>(q_row + pc * 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 4 * g + e;
          const uint4 kv = *reinterpret_cast<const uint4*>(k_tile + (row * RP + (pc ^ piece_swizzle<RP>(row))) * 16);
          acc[e] = dot_piece<DTYPE>(kv, qv, acc[e]);
        }
      }
    } else
#endif
    {
      // S^T = K Q^T on MFMA: lane (g, t) reads row t, pieces g*QP .. g*QP+QP-1
      const int ksw = piece_swizzle<RP>(t);
#pragma unroll
      for (int c = 0; c < QP; ++c) {
        const uint4 kp = *reinterpret_cast<const uint4*>(k_tile + (t * RP + ((g * QP + c) ^ ksw)) * 16);
        acc = mfma_qk<DTYPE>(kp, qr[c], acc);
      }
    }
    const int tile_tok = tok_begin + k * Tr::kChunk + wave * kTile;
    float s[4];  // s - m of the lane's 4 tokens (-inf past the piece)
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] = tile_tok + 4 * g + e < tok_end ? acc[e] * a.scale_log2 : kNegInf;
    // P = exp2(s - m), rounded to the MFMA input type; the sum uses the
    // rounded values so O / l is an exact convex combination of V rows.
    // A tile whose 16 tokens all count first keeps p = exp2(s - m) with m
    // unchanged when every head's tile sum lies in [2^-12, 2^12] (then no
    // p exceeds 2^12 and l stays far from underflow): no maximum, no
    // exchange of it and no rescale of O. Otherwise the tile is exact: the
    // head's maximum d of s - m moves m by max(d, 0) (by d while the head
    // has seen no token) and O, l are rescaled.
    float p[4];
    float lc = 0.f;
    bool kept = false;
    if (tile_tok + kTile <= tok_end) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[e] = to_f32<DTYPE>(from_f32<DTYPE>(__builtin_amdgcn_exp2f(s[e])));
        lc += p[e];
      }
      lc = rows_sum(lc);
      const bool out_of_range = !(lc <= kLazyMax && l_run + lc >= kLazyMin);  // NaN: out
      if (__builtin_amdgcn_ballot_w64(out_of_range) == 0) {
        l_run += lc;
        kept = true;
      }
    }
    if (!kept) {
      float mc = kNegInf;
#pragma unroll
      for (int e = 0; e < 4; ++e) mc = fmaxf(mc, s[e]);
      mc = rows_max(mc);  // head t's max over the tile: lanes t, t+16, t+32, t+48
      const bool seen = l_run > 0.f;
      const float shift = mc == kNegInf ? 0.f : seen ? fmaxf(mc, 0.f) : mc;
      const float alpha = seen ? __builtin_amdgcn_exp2f(-shift) : 0.f;  // O, l are 0 when unseen
      lc = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[e] = to_f32<DTYPE>(from_f32<DTYPE>(__builtin_amdgcn_exp2f(s[e] - shift)));
        lc += p[e];
      }
      lc = rows_sum(lc);
      l_run = l_run * alpha + lc;
      m_run += shift;
      // rescale O rows (head 4g+e takes the alpha of lane 4g+e)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float ar = __shfl(alpha, 4 * g + e);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) o[c][e] *= ar;
      }
    }
    if constexpr (kEarlyV) {
      s16x4 pa[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) pa[0][e] = static_cast<short>(from_f32<DTYPE>(p[e]));
      mfma_pv_operands<DTYPE, D, 1>(pa, vb, reinterpret_cast<f32x4(&)[1][D / 16]>(o));
    } else {
      mfma_pv<DTYPE, D>(p, v_tile, g, t, o);
    }
  };

  // Zeroes the V slots of tokens that were not loaded (P is 0 there, but
  // the pool row read in their place could hold NaN/Inf and 0 * NaN = NaN).
  auto zero_invalid_v = [&](int st, unsigned valid) __attribute__((always_inline)) {
    char* vdst = s_lds + wave * Tr::kWaveLds + st * Tr::kStageBytes + Tr::kTileBytes;
#pragma unroll
    for (int c = 0; c < L; ++c)
      if (!((valid >> c) & 1u))
        *reinterpret_cast<uint4*>(vdst + c * 1024 + lane * 16) = make_uint4(0, 0, 0, 0);
  };

  // ---- tile loop ---------------------------------------------------------
  // S = kStages buffers per wave. Chunk k's tile goes to stage k % S; at
  // step k the tile of chunk k+S-1 is issued into the stage chunk k-1 has
  // just released, then the wave waits until only the tiles of chunks
  // k+1 .. k+S-1 are in flight (vmcnt retires in order and the loop issues
  // no other vector memory instructions) and computes chunk k.
  constexpr int S = Tr::kStages;
  unsigned valid[S];
  auto step = [&](int k, auto st_c) __attribute__((always_inline)) {
    constexpr int ST = decltype(st_c)::value;
    constexpr int NX = (ST + S - 1) % S;
    if (k + S - 1 < n_chunks) valid[NX] = issue_tile(k + S - 1, IntC<NX>{});
    asm volatile("" ::: "memory");
    wait_vmcnt_groups<2 * L, S - 1>(n_chunks - 1 - k);
    asm volatile("" ::: "memory");
    // (only where a slot of this wave holds no token: a piece's last tile,
    // or a block id outside the pool; at every tile this cost c4 0.25 and
    // c5 0.6 us per layer call)
    if (__builtin_amdgcn_ballot_w64(valid[ST] != (1u << L) - 1u) != 0) zero_invalid_v(ST, valid[ST]);
    if constexpr (FUSED) {
      // the new token's row: last chunk, wave new_wave, row (tok_end - 1) % 16,
      // replaced when the slot is the token's table position (checked here,
      // long after the slot's load was issued)
      if (last_piece && k == n_chunks - 1 && wave == new_wave) {
        const int lt = tok_end - 1;
        const int id = s_ids[min((lt >> a.bs_log2) - first_blk, kIdCap - 1)];
        if (id >= 0 && new_slot == (static_cast<int64_t>(id) << a.bs_log2) + (lt & bs_mask) &&
            lane < 2 * RP) {
          const int r = (lt - tok_begin) % kTile;
          char* tile = s_lds + wave * Tr::kWaveLds + ST * Tr::kStageBytes + (lane < RP ? 0 : Tr::kTileBytes);
          *reinterpret_cast<uint4*>(tile + (r * RP + (new_pc ^ piece_swizzle<RP>(r))) * 16) = new_piece;
        }
      }
    }
    compute_tile(k, ST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the stage's LDS accesses are done
    asm volatile("" ::: "memory");
  };
  valid[0] = issue_tile(0, IntC<0>{});
  if constexpr (S > 2) {
    if (1 < n_chunks) valid[1] = issue_tile(1, IntC<1>{});
  }
  if constexpr (S > 3) {
    if (2 < n_chunks) valid[2] = issue_tile(2, IntC<2>{});
  }
  // Q (and the rotary and new rows) landed once wave 0's copies older than
  // these tiles are done.
  asm volatile("" ::: "memory");
  if (wave == 0) wait_vmcnt_groups<2 * L, S - 1>(min(S - 1, n_chunks));
  __syncthreads();  // Q rows visible to every wave
  {
    const char* q_row = s_lds + Tr::kQOffset + t * Tr::kRowBytes;
#pragma unroll
    for (int c = 0; c < QP; ++c) qr[c] = *reinterpret_cast<const uint4*>(q_row + (g * QP + c) * 16);
  }
  if constexpr (ROPE) {
    // RoPE of the Q operand in registers, by every wave: lane (g, t) holds
    // dims [g D/4, (g+1) D/4) of row t, and the other half of the row
    // (dims +D/2) sits in lane (g ^ 2, t) = lane ^ 32, one permlane32 swap
    // away; the cos / sin rows landed in LDS with the Q rows.
    const char* rope = s_lds + Tr::kRopeOffset;
#pragma unroll
    for (int c = 0; c < QP; ++c) {
      const int pc = g * QP + c;  // the 16-byte piece of the row
      const uint4 partner = swap_wave_halves(qr[c], lane);
      const uint4 cs = *reinterpret_cast<const uint4*>(rope + pc * 16);
      const uint4 sn = *reinterpret_cast<const uint4*>(rope + Tr::kRowBytes + pc * 16);
      qr[c] = rotate_chunk<DTYPE>(qr[c], partner, cs, sn, g < 2);
    }
  }
  if constexpr (FUSED) {
    if (last_piece) new_slot = *reinterpret_cast<const int64_t*>(s_lds + Tr::kSlotOffset);
    if (last_piece && wave == new_wave) {  // wave-uniform
      // the new rows, landed with the Q rows (the barrier above)
      if (new_lane) new_piece = *reinterpret_cast<const uint4*>(s_lds + Tr::kNewOffset + lane * 16);
      if constexpr (ROPE) {
        // RoPE of the new key row (lanes [0, RP)): chunk pc pairs with
        // chunk pc ^ RP/2 of the other half; cos / sin at its own dims
        uint4 partner;
        partner.x = __shfl_xor(new_piece.x, RP / 2);
        partner.y = __shfl_xor(new_piece.y, RP / 2);
        partner.z = __shfl_xor(new_piece.z, RP / 2);
        partner.w = __shfl_xor(new_piece.w, RP / 2);
        if (lane < RP) {
          const char* rope = s_lds + Tr::kRopeOffset;
          const uint4 c = *reinterpret_cast<const uint4*>(rope + lane * 16);
          const uint4 sn = *reinterpret_cast<const uint4*>(rope + Tr::kRowBytes + lane * 16);
          new_piece = rotate_chunk<DTYPE>(new_piece, partner, c, sn, lane < RP / 2);
        }
      }
      // the KV write of the new token (-1 skips), issued here rather than
      // after the tile loop, where the merge's wait for its stores would
      // also wait for this one (0.13 us of a c2 layer call). The tile copy
      // of the slot's own row may read the old row, the new one or a mix:
      // its LDS row is replaced with these rows before it is used, and no
      // other table entry of the batch reads the slot (the precondition).
      // Older than every tile copy, the store only makes the loop's vmcnt
      // waits wait for it too.
      if (new_lane && new_slot >= 0 && new_slot < a.total_slots) {
        const int64_t blk = new_slot >> a.bs_log2;
        const int64_t row = ((blk * a.num_kv_heads + h) << a.bs_log2) + (new_slot & bs_mask);
        char* dst = const_cast<char*>(lane < RP ? a.k_cache : a.v_cache) + row * Tr::kRowBytes;
        *reinterpret_cast<uint4*>(dst + new_pc * 16) = new_piece;
      }
    }
  }
  for (int k = 0; k < n_chunks; k += S) {
    step(k, IntC<0>{});
    if (k + 1 >= n_chunks) break;
    step(k + 1, IntC<1>{});
    if constexpr (S > 2) {
      if (k + 2 >= n_chunks) break;
      step(k + 2, IntC<2>{});
    }
    if constexpr (S > 3) {
      if (k + 3 >= n_chunks) break;
      step(k + 3, IntC<3>{});
    }
  }

  // ---- merge the waves ------------------------------------------------------
  // From here on thread (r, q) = (tid / 16, tid % 16) owns the dim pairs
  // (32j + 2q, 32j + 2q + 1), j < D/32, of query head r of the group: each
  // load or store instruction then covers 128 contiguous bytes per head.
  // Each wave parks its o rows and (max, sum) in its own tile buffers, free
  // once its loop is done (its copies and LDS reads have all completed), so
  // one barrier suffices and no wave waits for the others before writing.
  constexpr int NPAIR = Tr::kPairsPerThread;
  constexpr int OS = Tr::kORowStride;
  auto wave_o = [&](int w) { return reinterpret_cast<float*>(s_lds + w * Tr::kWaveLds); };  // [kMaxGroup][OS]
  auto wave_ms = [&](int w) { return wave_o(w) + kMaxGroup * OS; };  // max [kMaxGroup], sum [kMaxGroup]
  {
    float* my_o = wave_o(wave);
    if (g == 0) {
      // a head that saw no token has no reference: weight 0 in the merge
      wave_ms(wave)[t] = l_run > 0.f ? m_run : kNegInf;
      wave_ms(wave)[kMaxGroup + t] = l_run;
    }
    // all 16 accumulator rows (= query heads of the group; rows >= n_rep
    // are never read): unconditional, conflict-free stores
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
#pragma unroll
      for (int e = 0; e < 4; ++e) my_o[(4 * g + e) * OS + 16 * c + t] = o[c][e];
    }
  }
  __syncthreads();

  // One query head per thread: kWaves * 4 >= kMaxGroup >= n_rep.
  static_assert(kWaves * 4 >= kMaxGroup, "one head per epilogue thread");
  const int q = threadIdx.x & 15;
  const int r = threadIdx.x >> 4;
  const bool has_row = r < a.n_rep;
  const int64_t slot_base = (static_cast<int64_t>(b) * a.num_q_heads + h * a.n_rep) * a.max_parts;
  // (threads past the group's heads address head 0's row and store nothing)
  raw_t* const op = static_cast<raw_t*>(a.out) + b * a.out_stride_tok +
                    (h * a.n_rep + (has_row ? r : 0)) * a.out_stride_head + 2 * q;
  // this work group's partial of head r: (max, sum) and its dim pairs, as
  // stored (the partial O words: two fp32, or two values of the 16-bit
  // data type)
  uint64_t own_ml = 0;
  uint64_t own_ov[NPAIR];
#pragma unroll
  for (int j = 0; j < NPAIR; ++j) own_ov[j] = 0;
  if (has_row) {
    float mx = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, wave_ms(w)[r]);
    float sum = 0.f;
    float2 v[NPAIR];
#pragma unroll
    for (int j = 0; j < NPAIR; ++j) v[j] = make_float2(0.f, 0.f);
    // Straight-line LDS reads (one round trip): a wave with no token of the
    // partition has max -inf, sum 0 and o 0, and gets weight 0.
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = wave_ms(w)[r];
      const float f = mw == kNegInf ? 0.f : __builtin_amdgcn_exp2f(mw - mx);
      sum += wave_ms(w)[kMaxGroup + r] * f;
      const float* src = wave_o(w) + r * OS + 2 * q;
#pragma unroll
      for (int j = 0; j < NPAIR; ++j) {
        const float2 x = *reinterpret_cast<const float2*>(src + 32 * j);
        v[j].x += x.x * f;
        v[j].y += x.y * f;
      }
    }
    // > 0: the wave whose reference is mx has l > 2^-12 (every kept tile
    // leaves l at least that, an exact one at least 1)
    const float inv = 1.f / sum;
    if (n_parts == 1) {
#pragma unroll
      for (int j = 0; j < NPAIR; ++j) {
        op[32 * j] = from_f32<DTYPE>(v[j].x * inv);
        op[32 * j + 1] = from_f32<DTYPE>(v[j].y * inv);
      }
    } else {
      own_ml = pack_f32x2(mx, sum);
#pragma unroll
      for (int j = 0; j < NPAIR; ++j) {
        if constexpr (kPartials16)  // dims 2q + 32j, +1 as two 16-bit values
          own_ov[j] = static_cast<uint32_t>(from_f32<DTYPE>(v[j].x * inv)) |
                      (static_cast<uint32_t>(from_f32<DTYPE>(v[j].y * inv)) << 16);
        else
          own_ov[j] = pack_f32x2(v[j].x * inv, v[j].y * inv);
      }
    }
  }
  if (n_parts == 1) return;

  // ---- cross-partition merge by the last work group --------------------
  auto ov_lo = [](uint64_t x) -> float {
    if constexpr (kPartials16) return to_f32<DTYPE>(static_cast<uint16_t>(x));
    else return unpack_lo(x);
  };
  auto ov_hi = [](uint64_t x) -> float {
    if constexpr (kPartials16) return to_f32<DTYPE>(static_cast<uint16_t>(x >> 16));
    else return unpack_hi(x);
  };
  if (has_row) {
    const int64_t slot = slot_base + static_cast<int64_t>(r) * a.max_parts + part;
#pragma unroll
    for (int j = 0; j < NPAIR; ++j) {
      if constexpr (kPartials16)
        store_coherent_u32(reinterpret_cast<uint32_t*>(a.ws_o) + slot * (D / 2) + q + 16 * j,
                           static_cast<uint32_t>(own_ov[j]));
      else
        store_coherent_u64(reinterpret_cast<uint64_t*>(a.ws_o + slot * D + 2 * q) + 16 * j, own_ov[j]);
    }
    if (q == 0) store_coherent_u64(reinterpret_cast<uint64_t*>(a.ws_ml) + slot, own_ml);
  }
  // The partials above are device-coherent stores; once every wave has
  // seen them acknowledged (vmcnt(0)), the counter increment publishes
  // them. The work group that completes the count reads the other
  // groups' partials with device-coherent loads. No L2 writeback or
  // invalidate is involved.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&a.counters[b * a.num_kv_heads + h], 1,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == n_parts - 1;
  }
  __syncthreads();
  if (!s_last) return;
  // Log-sum-exp over the partitions in rounds: every thread issues the
  // (max, sum) pairs of its head and its dims of the partials of a round
  // together (one memory round trip per round; the round size is the
  // smallest of 4, 8, kMergeRound that fits, so few loads are wasted), then
  // folds them into a running (max, sum, o) with one rescale per round.
  // The merging group's own partial comes from its registers (the bits it
  // stored), not from memory.
  if (has_row) {
    const int64_t slot0 = slot_base + static_cast<int64_t>(r) * a.max_parts;
    float m_all = kNegInf, l_all = 0.f;
    float2 acc[NPAIR];
#pragma unroll
    for (int j = 0; j < NPAIR; ++j) acc[j] = make_float2(0.f, 0.f);
    // Folds partitions [p0, p0 + np), np <= RR.
    auto fold = [&](auto rr_c, int p0, int np) __attribute__((always_inline)) {
      constexpr int RR = decltype(rr_c)::value;
      // Straight-line loads (entries past the last partition re-read it and
      // get weight 0), so the whole round is in flight before the first use.
      uint64_t ml[RR];
      uint64_t ov[RR][NPAIR];
#pragma unroll
      for (int pp = 0; pp < RR; ++pp) {
        const int p = p0 + min(pp, np - 1);
        if (p == part) {  // work-group uniform
          ml[pp] = own_ml;
#pragma unroll
          for (int j = 0; j < NPAIR; ++j) ov[pp][j] = own_ov[j];
          continue;
        }
        const int64_t slot = slot0 + p;
        ml[pp] = load_coherent_u64(reinterpret_cast<const uint64_t*>(a.ws_ml) + slot);
        if constexpr (kPartials16) {
          const uint32_t* src = reinterpret_cast<const uint32_t*>(a.ws_o) + slot * (D / 2) + q;
#pragma unroll
          for (int j = 0; j < NPAIR; ++j) ov[pp][j] = load_coherent_u32(src + 16 * j);
        } else {
          const uint64_t* src = reinterpret_cast<const uint64_t*>(a.ws_o + slot * D + 2 * q);
#pragma unroll
          for (int j = 0; j < NPAIR; ++j) ov[pp][j] = load_coherent_u64(src + 16 * j);
        }
      }
      float m_round = m_all;
#pragma unroll
      for (int pp = 0; pp < RR; ++pp) m_round = fmaxf(m_round, unpack_lo(ml[pp]));
      const float rescale = __builtin_amdgcn_exp2f(m_all - m_round);  // 0 on the first round
      l_all *= rescale;
#pragma unroll
      for (int j = 0; j < NPAIR; ++j) {
        acc[j].x *= rescale;
        acc[j].y *= rescale;
      }
#pragma unroll
      for (int pp = 0; pp < RR; ++pp) {
        const float w =
            pp < np ? unpack_hi(ml[pp]) * __builtin_amdgcn_exp2f(unpack_lo(ml[pp]) - m_round) : 0.f;
        l_all += w;
#pragma unroll
        for (int j = 0; j < NPAIR; ++j) {
          acc[j].x += w * ov_lo(ov[pp][j]);
          acc[j].y += w * ov_hi(ov[pp][j]);
        }
      }
      m_all = m_round;
    };
    constexpr int RMAX = Tr::kMergeRound;
    for (int p0 = 0; p0 < n_parts; p0 += RMAX) {
      const int np = min(RMAX, n_parts - p0);
      if (np <= 4) fold(IntC<4>{}, p0, np);
      else if (RMAX <= 8 || np <= 8) fold(IntC<(RMAX < 8 ? RMAX : 8)>{}, p0, np);
      else fold(IntC<RMAX>{}, p0, np);
    }
    const float inv = 1.f / l_all;
#pragma unroll
    for (int j = 0; j < NPAIR; ++j) {
      op[32 * j] = from_f32<DTYPE>(acc[j].x * inv);
      op[32 * j + 1] = from_f32<DTYPE>(acc[j].y * inv);
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
  int32_t num_seqs, max_blocks, bs_log2, num_kv_heads, groups_per_cu, cu_count;
  int32_t fixed_part_tokens;  // > 0: ids stride for this piece bound, unused slots marked
  int64_t num_blocks;
  int32_t* work;      // [work_cap][8]: one entry per work group (launch slot)
  int64_t work_cap;   // entries
  int32_t* ids;
  int64_t ids_cap;
  int32_t* counters;
  int32_t* status;
};

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kDealMax = 1024;       // work groups sorted and dealt to CUs in shared memory
constexpr int kPlanSeqCache = 4096;  // kv lengths held in shared memory
constexpr int kWaveSearchSeqs = 256; // one wave runs the piece-bound search up to this batch
constexpr int kWavePlanSeqs = 64;     // decode_plan_wave_kernel (one sequence per lane) up to this batch
constexpr int kWavePlanWaves = 4;     // its waves (a power of 2)
constexpr int64_t kFusedTableEntries = 8192;  // plan and ids in one launch up to this table size
constexpr int64_t kFusedSlots = 4096;         // ... and this many slots (one wave each)
constexpr int kIdsThreads = 256;     // block-id kernel: threads per work group
static_assert(kPlanThreads == kDealMax, "the deal holds one group (and one bucket) per thread");

// Value-returning min / max: std::min / std::max return a reference, and
// a reference to one of two temporaries makes the compiler keep both on
// the stack to select an address.
template <typename T> __device__ inline T vmin(T x, T y) { return y < x ? y : x; }
template <typename T> __device__ inline T vmax(T x, T y) { return x < y ? y : x; }

// Wave-wide scans on DPP lane moves (a few cycles each, against an LDS
// round trip for a shuffle). DPP controls: row_shr:n (0x110 + n) reads lane
// i - n of the same 16-lane row, row_shl:n (0x100 + n) lane i + n, row_ror:n
// (0x120 + n) rotates the row, quad_perm (0x00-0xFF) permutes within 4
// lanes, row_bcast:15 (0x142) / row_bcast:31 (0x143) read lane 15 of the
// previous row / lane 31. A lane whose source lies outside its row, or
// whose row is masked off, gets `fill`.
template <int CTRL, int ROW_MASK = 0xF>
__device__ inline int dpp(int fill, int v) {
  return __builtin_amdgcn_update_dpp(fill, v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ inline int64_t dpp64(int64_t v) {
  const int lo = dpp<CTRL, ROW_MASK>(0, static_cast<int>(v));
  const int hi = dpp<CTRL, ROW_MASK>(0, static_cast<int>(v >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                              static_cast<uint32_t>(lo));
}
// Inclusive scan over the 64 lanes (all active): within each row by
// shifts 1, 2, 4, 8, then row totals carried by the two broadcasts.
template <typename Op>
__device__ inline int wave_scan(int v, int identity, Op op) {
  v = op(v, dpp<0x111>(identity, v));
  v = op(v, dpp<0x112>(identity, v));
  v = op(v, dpp<0x114>(identity, v));
  v = op(v, dpp<0x118>(identity, v));
  v = op(v, dpp<0x142, 0xA>(identity, v));
  v = op(v, dpp<0x143, 0xC>(identity, v));
  return v;
}
__device__ inline int wave_scan_sum(int v) {
  return wave_scan(v, 0, [](int x, int y) { return x + y; });
}
__device__ inline int wave_sum(int v) { return __builtin_amdgcn_readlane(wave_scan_sum(v), 63); }
__device__ inline int wave_max(int v) {
  return __builtin_amdgcn_readlane(wave_scan(v, INT_MIN, [](int x, int y) { return max(x, y); }), 63);
}
__device__ inline int wave_min(int v) {
  return __builtin_amdgcn_readlane(wave_scan(v, INT_MAX, [](int x, int y) { return min(x, y); }), 63);
}
__device__ inline int64_t wave_sum64(int64_t v) {
  v += dpp64<0x111>(v);
  v += dpp64<0x112>(v);
  v += dpp64<0x114>(v);
  v += dpp64<0x118>(v);
  v += dpp64<0x142, 0xA>(v);
  v += dpp64<0x143, 0xC>(v);
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(v), 63);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(v >> 32), 63);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
// Work-group sum of one value per thread. The trailing barrier lets the
// next call reuse the scratch.
__device__ int64_t block_sum64(int64_t v, int64_t* scratch) {
  v = wave_sum64(v);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  const int lane = threadIdx.x & 63;  // lane w reads wave w's sum
  const int64_t total = wave_sum64(lane < kPlanWaves ? scratch[lane] : 0);
  __syncthreads();
  return total;
}

// Block ids stored per work group for pieces of at most `part_tokens`
// tokens: a piece spans at most ceil(P / bs) + 1 table entries; rounded up
// to a multiple of 4 so every list is 16-byte aligned.
__host__ __device__ inline int ids_per_item(int64_t part_tokens, int bs_log2) {
  const int64_t n = ((part_tokens + (int64_t(1) << bs_log2) - 1) >> bs_log2) + 1;
  return static_cast<int>((n + 3) / 4 * 4);
}

// Token range of piece j of a sequence of kv tokens cut into np pieces:
// equal shares of its 16-token tiles (32-bit arithmetic when j * tiles
// fits, which holds for every table of fewer than 2^16 tiles).
__device__ inline int2 piece_range(int kv, int np, int j) {
  const int tiles = (kv + kTile - 1) / kTile;
  int t0, t1;
  if (tiles < (1 << 16)) {
    t0 = static_cast<int>(static_cast<uint32_t>(j) * tiles / static_cast<uint32_t>(np)) * kTile;
    t1 = static_cast<int>(static_cast<uint32_t>(j + 1) * tiles / static_cast<uint32_t>(np)) * kTile;
  } else {
    t0 = static_cast<int>(static_cast<int64_t>(j) * tiles / np) * kTile;
    t1 = static_cast<int>(static_cast<int64_t>(j + 1) * tiles / np) * kTile;
  }
  return make_int2(t0, min(kv, t1));
}

// Step 2 of the plan, shared by both plan kernels: the resident target and
// the range the piece bound L (in 16-token tiles) is searched in.
//   Resident slots to fill: 2 per CU when there is at most one (sequence,
//   kv head) unit per CU -- fewer, longer pieces per CU stream at a
//   steadier rate per CU than three or four (measured on c2/c3-like
//   batches), and the split-K merge has fewer partials -- otherwise up to
//   kManyUnitsPerCU (3 beat the 4 that LDS allows at D=64 on the c4 batch).
//   A piece spans at most kIdCap table entries (they are staged in LDS):
//   L <= l_cap, hard. At least one tile per wave per piece and at most
//   kMaxParts pieces per sequence: L >= l_min, soft.
// n / d for n >= 0, d > 0: a 32-bit division when both fit (the usual
// case; the 64-bit expansion is a long dependent chain).
__device__ inline int64_t div_nonneg(int64_t n, int64_t d) {
  if (((n | d) >> 32) == 0) return static_cast<uint32_t>(n) / static_cast<uint32_t>(d);
  return n / d;
}

struct PieceRules {
  int64_t target;
  int l_cap, l_min, l_top, l_fair;
};
__device__ inline PieceRules piece_rules(int groups_per_cu, int cu_count, int bs_log2, int64_t units,
                                         int64_t total_tiles, int most_tiles, int hkv) {
  PieceRules r;
  const int per_cu = units <= cu_count ? vmin(kFewUnitsPerCU, vmax(1, groups_per_cu))
                                       : vmin(kManyUnitsPerCU, vmax(1, groups_per_cu));
  r.target = static_cast<int64_t>(per_cu) * vmax(1, cu_count);
  r.l_cap = static_cast<int>(vmax<int64_t>(
      1, vmin<int64_t>(INT_MAX / 32, ((static_cast<int64_t>(kIdCap - 1)) << bs_log2) / kTile)));
  r.l_min = vmin(r.l_cap, vmax(kWaves, (most_tiles + kMaxParts - 1) / kMaxParts));
  r.l_top = vmin(r.l_cap, vmax(r.l_min, most_tiles));
  r.l_fair = static_cast<int>(vmin<int64_t>(
      r.l_cap, vmax<int64_t>(r.l_min, div_nonneg(total_tiles * hkv + r.target - 1, r.target))));
  return r;
}

// The smallest l in [l_min, l_top] whose groups fit the target (see
// decode_plan_kernel, step 2). groups(l) = hkv * sum ceil(tiles_b / l)
// lies in [hkv * total / l, hkv * total / l + units), so no l below
// ceil(hkv * total / target) fits and every l from
// ceil(hkv * total / (target - units)) on does: the search runs between
// the two (a handful of steps, not log2(l_top)). `known` holds groups(l)
// for the returned l when the search evaluated it, else -1.
template <typename F>
__device__ inline int pick_piece_bound(const PieceRules& r, int64_t units, int64_t total_tiles, int hkv,
                                       F&& groups_at, int64_t& known) {
  known = -1;
  int lo = vmin(r.l_fair, r.l_top), hi = r.l_top;
  bool top_fits = false;
  if (r.target > units) {
    const int64_t l_fit = div_nonneg(total_tiles * hkv + (r.target - units) - 1, r.target - units);
    if (l_fit <= r.l_top) {
      hi = vmax(lo, static_cast<int>(l_fit));
      top_fits = true;
    }
  }
  if (!top_fits) {
    known = groups_at(r.l_top);
    if (known > r.target) {  // more sequences than slots: several rounds
      known = -1;
      return r.l_fair;
    }
  }
  while (lo < hi) {
    const int mid = lo + (hi - lo) / 2;
    const int64_t g = groups_at(mid);
    if (g <= r.target) {
      hi = mid;
      known = g;
    } else {
      lo = mid + 1;
    }
  }
  if (lo > 2 * r.l_fair) {
    known = -1;
    return vmax(r.l_min, vmin(r.l_cap, 2 * r.l_fair));
  }
  return lo;
}

// One work group builds the per-step decode plan:
//   1. validates kv_len (and, with the block ids of step 5, every table
//      entry a sequence reads);
//   2. picks the piece bound L (16-token tiles): the smallest that keeps
//      the (sequence, kv head, piece) work groups within one dispatch round
//      (groups_per_cu x cu_count), so every group is resident at once --
//      unless that needs pieces over twice the fair share of the slots (a
//      few very long sequences): then pieces of about the fair share run in
//      several rounds and the dispatcher balances them;
//   3. cuts each sequence into ceil(tiles / L) pieces of equal tile counts;
//   4. when the groups fit one round, sorts them by size and deals them to
//      launch slots in snake order over the CUs: work group i of a resident
//      grid runs on the same CU as group i + cu_count (dispatch is
//      round-robin), so slot s lands on CU "s mod cu_count" and the CUs
//      carry near-equal bytes (a CU streams at a bounded rate, so the most
//      loaded one sets the kernel time);
//   5. stores each slot's entry (seq, kv head, piece, pieces, token range),
//      zeroes the merge counters, and publishes the ids per slot for
//      decode_ids_kernel (or checks the table itself when the list does
//      not fit: the plan is then unusable and says so).
// It runs once per engine step, so its latency is what counts: the kv
// lengths stay in shared memory and the search and scans use wave
// shuffles. The block ids (step 5) are written by decode_ids_kernel, which
// spreads them over many CUs (one CU streams only ~20 GB/s).
template <typename KV, typename BT>
__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(PlanArgs a) {
  __shared__ int s_kv[kPlanSeqCache];     // kv_len, or 0 for an invalid length
  __shared__ int64_t s_red[kPlanWaves];
  __shared__ int64_t s_tiles[kPlanWaves];
  __shared__ int s_red5[5][kPlanWaves];  // live sequences, most tiles, least kv, bad kv, short table
  __shared__ int s_wsum[2][kPlanWaves];
  __shared__ int s_max_parts;
  __shared__ int s_lb;
  __shared__ int64_t s_groups;
  __shared__ uint32_t s_key[2][kDealMax];                 // the deal's bucket counts and starts
  __shared__ int s_item_b[kDealMax], s_item_j[kDealMax];  // items (sequence, piece) when dealt
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  if (tid == 0) s_max_parts = 0;

  const KV* kvp = static_cast<const KV*>(a.kv_len);
  const BT* btp = static_cast<const BT*>(a.block_table);
  const int64_t bs = int64_t(1) << a.bs_log2;
  const int hkv = a.num_kv_heads;
  const bool cached = a.num_seqs <= kPlanSeqCache;
  auto clean_len = [&](int64_t kv) -> int {  // 0 for a length no piece reads
    const bool ok = kv >= 1 && (kv + bs - 1) / bs <= a.max_blocks && kv <= INT_MAX / 2;
    return ok ? static_cast<int>(kv) : 0;
  };
  auto kv_of = [&](int b) -> int {
    return cached ? s_kv[b] : clean_len(static_cast<int64_t>(kvp[b]));
  };
  auto tiles_of = [&](int b) -> int { return (kv_of(b) + kTile - 1) / kTile; };

  // ---- 1. lengths
  {
    int64_t tiles = 0;
    int seqs = 0, max_tiles = 0, min_kv = INT_MAX, bad_kv = 0, short_table = 0;
    for (int b = tid; b < a.num_seqs; b += kPlanThreads) {
      const int64_t kv = static_cast<int64_t>(kvp[b]);
      min_kv = min(min_kv, static_cast<int>(vmax<int64_t>(vmin<int64_t>(kv, INT_MAX), INT_MIN)));
      const int c = clean_len(kv);
      bad_kv += kv < 1;
      short_table += kv >= 1 && c == 0;
      if (cached) s_kv[b] = c;
      const int t = (c + kTile - 1) / kTile;
      tiles += t;
      max_tiles = max(max_tiles, t);
      seqs += c > 0;
    }
    tiles = wave_sum64(tiles);
    seqs = wave_sum(seqs);
    max_tiles = wave_max(max_tiles);
    min_kv = wave_min(min_kv);
    bad_kv = wave_sum(bad_kv);
    short_table = wave_sum(short_table);
    if (lane == 0) {
      s_tiles[wave] = tiles;
      s_red5[0][wave] = seqs;
      s_red5[1][wave] = max_tiles;
      s_red5[2][wave] = min_kv;
      s_red5[3][wave] = bad_kv;
      s_red5[4][wave] = short_table;
    }
  }
  __syncthreads();
  // the waves' totals: lane w reads wave w's, then one wave reduction per
  // value (16 serial broadcast reads per value and thread kept the CU's LDS
  // busy for about 1500 cycles)
  int64_t total_tiles, live_seqs;
  int most_tiles, least_kv, bad_kv, short_table;
  {
    const bool in = lane < kPlanWaves;
    total_tiles = wave_sum64(in ? s_tiles[lane] : 0);
    live_seqs = wave_sum(in ? s_red5[0][lane] : 0);
    most_tiles = wave_max(in ? s_red5[1][lane] : 0);
    least_kv = wave_min(in ? s_red5[2][lane] : INT_MAX);
    bad_kv = wave_sum(in ? s_red5[3][lane] : 0);
    short_table = wave_sum(in ? s_red5[4][lane] : 0);
  }
  const int64_t units = live_seqs * hkv;  // (sequence, kv head) pairs

  // ---- 2. piece bound L (tiles)
  const PieceRules rules =
      piece_rules(a.groups_per_cu, a.cu_count, a.bs_log2, units, total_tiles, most_tiles, hkv);
  const int64_t target = rules.target;
  auto pick = [&](auto&& groups_at, int64_t& known) -> int {
    return pick_piece_bound(rules, units, total_tiles, hkv, groups_at, known);
  };
  int lb;
  int64_t num_groups;
  if (cached && a.num_seqs <= kWaveSearchSeqs) {
    // one wave, no barriers in the search; the lane's (at most 4) tile
    // counts stay in registers, and the count sums in 32 bits while it fits
    // (a search step is then a few divisions and one 32-bit wave sum)
    if (wave == 0) {
      static_assert(kWaveSearchSeqs <= 4 * 64, "4 sequences per lane");
      int t4[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) t4[k] = lane + 64 * k < a.num_seqs ? tiles_of(lane + 64 * k) : 0;
      const bool narrow = static_cast<int64_t>(a.num_seqs) * most_tiles < (int64_t(1) << 30);
      const int per_lane = (a.num_seqs + 63) / 64;  // wave-uniform, at most 4
      auto groups_wave = [&](int l) -> int64_t {
        int n = (t4[0] + l - 1) / l;
#pragma unroll
        for (int k = 1; k < 4; ++k)
          if (k < per_lane) n += (t4[k] + l - 1) / l;
        return (narrow ? static_cast<int64_t>(wave_sum(n)) : wave_sum64(n)) * hkv;
      };
      int64_t g;
      const int l = pick(groups_wave, g);
      if (g < 0) g = groups_wave(l);
      if (lane == 0) {
        s_lb = l;
        s_groups = g;
      }
    }
    __syncthreads();
    lb = s_lb;
    num_groups = s_groups;
  } else {
    auto groups_block = [&](int l) -> int64_t {  // uniform call: every thread
      int64_t n = 0;
      for (int b = tid; b < a.num_seqs; b += kPlanThreads) n += (tiles_of(b) + l - 1) / l;
      return block_sum64(n, s_red) * hkv;
    };
    lb = pick(groups_block, num_groups);
    if (num_groups < 0) num_groups = groups_block(lb);
  }
  const int part_tokens = lb * kTile;

  // ---- 3. items (sequence, piece) in sequence order
  const bool deal = num_groups <= kDealMax && num_groups <= target && a.cu_count > 0;
  const int64_t used_groups = vmin<int64_t>(num_groups, a.work_cap);
  int64_t running = 0;
  int parity = 0;
  for (int base = 0; base < a.num_seqs; base += kPlanThreads, parity ^= 1) {
    const int b = base + tid;
    const int np = b < a.num_seqs ? (tiles_of(b) + lb - 1) / lb : 0;
    const int most = wave_max(np);
    if (lane == 0 && most > 0) atomicMax(&s_max_parts, most);
    // exclusive scan of np: inclusive within the wave, then wave totals
    const int incl = wave_scan_sum(np);
    if (lane == 63) s_wsum[parity][wave] = incl;
    __syncthreads();  // alternate buffers: the next chunk writes the other one
    // earlier waves' and all waves' totals: lane w holds wave w's, scanned
    const int wscan = wave_scan_sum(lane < kPlanWaves ? s_wsum[parity][lane] : 0);
    const int before = wave == 0 ? 0 : __builtin_amdgcn_readlane(wscan, __builtin_amdgcn_readfirstlane(wave - 1));
    const int chunk = __builtin_amdgcn_readlane(wscan, kPlanWaves - 1);
    const int64_t start = running + before + incl - np;
    if (deal) {
      // items < num_groups / hkv <= kDealMax; the wave-uniform trip count
      // (the wave's most pieces) keeps this a scalar loop with one masked
      // pair of LDS writes per step, not a divergent per-lane loop
      const int first = static_cast<int>(start);
      for (int j = 0; j < most; ++j)
        if (j < np && first + j < kDealMax) {
          s_item_b[first + j] = b;
          s_item_j[first + j] = j;
        }
    } else {
      for (int j = 0; j < np; ++j) {
        const int64_t item = start + j;
        const int2 r = piece_range(kv_of(b), np, j);
        for (int h = 0; h < hkv; ++h) {
          const int64_t slot = item * hkv + h;
          if (slot < a.work_cap) {
            int4* w = reinterpret_cast<int4*>(a.work + 8 * slot);
            w[0] = make_int4(b, h, j, np);
            w[1] = make_int4(r.x, r.y, 0, 0);
          }
        }
      }
    }
    running += chunk;
  }
  // the deal's buckets: (L - size) >> shift for piece sizes 1..L tiles,
  // cleared here so the items barrier covers it
  int* s_count = reinterpret_cast<int*>(s_key[0]);  // groups per bucket
  int* s_start = reinterpret_cast<int*>(s_key[1]);  // first position of each bucket
  int shift = 0;
  while ((lb >> shift) >= kDealMax) ++shift;
  const int buckets = ((lb - 1) >> shift) + 1;  // <= kDealMax
  if (deal && tid < buckets) s_count[tid] = 0;
  __syncthreads();  // items complete

  // ---- 4. deal: order the groups by size (descending) and place sorted
  // position p in slot r * cu_count + c (round r = p / cu_count), forward
  // or backward over c by round parity, ending forward so the last
  // partial round fills slots [r * cu_count, r * cu_count + rem).
  // Counting sort: bucket k = (L - size) >> shift of at most kDealMax
  // buckets (exact sizes for L < kDealMax tiles), position = the bucket's
  // start + the group's arrival order in it (groups of one size are
  // interchangeable here; the results never depend on the placement).
  if (deal) {
    int bucket = 0, within = 0, b = 0, h = 0, j = 0, np = 0;
    int2 r = make_int2(0, 0);
    if (tid < num_groups) {
      const int item = tid / hkv;
      h = tid - item * hkv;
      b = s_item_b[item];
      j = s_item_j[item];
      np = (tiles_of(b) + lb - 1) / lb;
      r = piece_range(kv_of(b), np, j);
      const int size = vmin((r.y - r.x + kTile - 1) / kTile, lb);
      bucket = (lb - size) >> shift;
      within = atomicAdd(&s_count[bucket], 1);
    }
    __syncthreads();
    // exclusive scan of the bucket counts, one bucket per thread: in one
    // wave when the buckets fit it (L <= 64 tiles), else over the block
    if (buckets <= 64) {
      if (wave == 0) {
        const int cnt = lane < buckets ? s_count[lane] : 0;
        s_start[lane] = wave_scan_sum(cnt) - cnt;
      }
    } else {
      const int cnt = tid < buckets ? s_count[tid] : 0;
      const int incl = wave_scan_sum(cnt);
      if (lane == 63) s_wsum[0][wave] = incl;
      __syncthreads();
      const int wscan = wave_scan_sum(lane < kPlanWaves ? s_wsum[0][lane] : 0);
      const int before = wave == 0 ? 0 : __builtin_amdgcn_readlane(wscan, __builtin_amdgcn_readfirstlane(wave - 1));
      s_start[tid] = before + incl - cnt;
    }
    __syncthreads();
    if (tid < num_groups) {
      const int pos = s_start[bucket] + within;
      const int cus = a.cu_count;
      const int rounds = static_cast<int>((num_groups + cus - 1) / cus);
      const int rd = pos / cus, c = pos - rd * cus;
      const bool forward = ((rounds - 1 - rd) & 1) == 0;
      const int slot = rd * cus + (forward ? c : cus - 1 - c);
      if (slot < a.work_cap) {
        int4* w = reinterpret_cast<int4*>(a.work + 8 * slot);
        w[0] = make_int4(b, h, j, np);
        w[1] = make_int4(r.x, r.y, 0, 0);
      }
    }
  }

  // ---- 5. block ids per slot: decode_ids_kernel, when the list fits.
  // With a fixed piece bound (a launch of fixed size, e.g. in a captured
  // graph) the id lists have that bound's stride, and the slots past the
  // last work group get an entry with sequence -1, which the decode kernel
  // skips.
  const bool fixed = a.fixed_part_tokens > 0;
  const int per_item = ids_per_item(fixed ? a.fixed_part_tokens : part_tokens, a.bs_log2);
  const int64_t n_ids = used_groups * per_item;
  const bool listed = used_groups == num_groups && n_ids <= a.ids_cap &&
                      n_ids <= INT_MAX &&
                      (!fixed || part_tokens <= a.fixed_part_tokens);
  // A plan whose id lists do not fit is unusable: every slot is marked
  // unused, so a launch of it does nothing (no piece runs without its ids).
  __syncthreads();  // the entries of steps 3-4 are written
  if (fixed || !listed) {
    for (int64_t slot = listed ? used_groups + tid : tid; slot < a.work_cap; slot += kPlanThreads) {
      int4* w = reinterpret_cast<int4*>(a.work + 8 * slot);
      w[0] = make_int4(-1, 0, 0, 0);
      w[1] = make_int4(0, 0, 0, 0);
    }
  }
  int64_t bad = 0;
  if (!listed) {  // uniform
    const int64_t n = static_cast<int64_t>(a.num_seqs) * a.max_blocks;
    for (int64_t i = tid; i < n; i += kPlanThreads) {
      const int64_t b = i / a.max_blocks;
      const int64_t j = i - b * a.max_blocks;
      if (j < (kv_of(static_cast<int>(b)) + bs - 1) / bs) {
        const int64_t blk = static_cast<int64_t>(btp[b * a.bt_stride + j]);
        bad += (blk < 0 || blk >= a.num_blocks);
      }
    }
    bad = block_sum64(bad, s_red);
  }
  const int64_t nc = static_cast<int64_t>(a.num_seqs) * hkv;
  for (int64_t i = tid; i < nc; i += kPlanThreads) a.counters[i] = 0;
  __syncthreads();
  if (tid == 0) {
    a.status[MV_PLAN_NUM_ITEMS] = static_cast<int32_t>(vmin<int64_t>(num_groups, INT_MAX));
    a.status[MV_PLAN_BAD_KV_LEN] = bad_kv;
    a.status[MV_PLAN_INSUFFICIENT] = short_table;
    a.status[MV_PLAN_BAD_BLOCK] = static_cast<int32_t>(vmin<int64_t>(bad, INT_MAX));  // the id kernel adds its count
    a.status[MV_PLAN_MAX_PARTS] = s_max_parts;
    a.status[MV_PLAN_MIN_KV_LEN] = a.num_seqs > 0 ? least_kv : 0;
    a.status[MV_PLAN_PARTITION_TOKENS] = part_tokens;
    a.status[MV_PLAN_IDS_PER_ITEM] = listed ? per_item : -1;  // -1: no list this step
  }
}

// Slot s's block-id list (step 5 of the plan): ids[s * n, (s + 1) * n) with
// n = per_item (a multiple of 4, at most kIdCap) holds the pool blocks of
// its piece in entries [0, span) and -1 for an entry outside the pool; -1
// fills the rest of the last group of four. Entries past that are not
// written: the decode kernel uses only [0, span) (with a fixed piece bound
// n is the widest piece's span, so most of each list is never written).
// One wave writes the list, 4 ids per lane per pass (at most 2 passes of
// 256). Returns this lane's count of bad entries among the reads of a kv
// head 0 piece's own blocks (a block belongs to the one piece that holds
// its first token, so over all slots each needed table entry counts once).
template <typename BT>
__device__ inline int write_slot_ids(const BT* btp, int64_t bt_stride, int num_seqs, int max_blocks,
                                     int64_t num_blocks, int bs_log2, int per_item, int32_t* ids,
                                     int64_t slot, int4 w0, int4 w1, int lane) {
  const int first = w1.x >> bs_log2;
  const int last = (w1.y - 1) >> bs_log2;
  // the bounds hold for every entry the plan writes
  const bool seq_ok = w0.x >= 0 && w0.x < num_seqs;
  const BT* row = btp + (seq_ok ? static_cast<int64_t>(w0.x) * bt_stride : 0);
  int4* out = reinterpret_cast<int4*>(ids + slot * per_item);
  const int span = seq_ok ? vmax(0, last - first + 1) : 0;
  const int n_write = vmin(per_item, (span + 3) & ~3);
  int bad = 0;
  for (int k0 = 4 * lane; k0 < n_write; k0 += 4 * 64) {
    int32_t v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = first + k0 + e;
      const bool read = seq_ok && m <= last && m >= 0 && m < max_blocks;
      const int64_t blk = read ? static_cast<int64_t>(row[m]) : -1;
      const bool in_pool = blk >= 0 && blk < num_blocks;
      bad += read && w0.y == 0 && (static_cast<int64_t>(m) << bs_log2) >= w1.x && !in_pool;
      v[e] = in_pool ? static_cast<int32_t>(blk) : -1;
    }
    out[k0 >> 2] = make_int4(v[0], v[1], v[2], v[3]);
  }
  return bad;
}

struct IdsArgs {
  const void* block_table;
  int64_t bt_stride;
  int32_t num_seqs, max_blocks;
  const int32_t* work;
  int64_t work_cap;
  int32_t* ids;
  int32_t* status;
  int64_t num_blocks;
  int32_t bs_log2;
};

// Step 5 of the plan, over many CUs, after a plan kernel: one wave per slot
// (write_slot_ids). The slot follows from blockIdx and the wave alone, so
// its work entry loads beside the status word: two dependent round trips
// (entry and status, then the table) before the stores. The bad entries
// counted are added to status[MV_PLAN_BAD_BLOCK].
template <typename BT>
__global__ __launch_bounds__(kIdsThreads) void decode_ids_kernel(IdsArgs a) {
  constexpr int kSlotsPerGroup = kIdsThreads / 64;
  const int lane = threadIdx.x & 63;
  const BT* btp = static_cast<const BT*>(a.block_table);
  int bad = 0;
  for (int64_t slot = static_cast<int64_t>(blockIdx.x) * kSlotsPerGroup + (threadIdx.x >> 6);
       slot < a.work_cap; slot += static_cast<int64_t>(gridDim.x) * kSlotsPerGroup) {
    const int4 w0 = reinterpret_cast<const int4*>(a.work + 8 * slot)[0];
    const int4 w1 = reinterpret_cast<const int4*>(a.work + 8 * slot)[1];
    const int per_item = a.status[MV_PLAN_IDS_PER_ITEM];  // -1: no list this step
    const int groups = a.status[MV_PLAN_NUM_ITEMS];
    if (per_item <= 0 || slot >= groups) break;  // uniform per wave; later slots are larger
    bad += write_slot_ids(btp, a.bt_stride, a.num_seqs, a.max_blocks, a.num_blocks, a.bs_log2, per_item,
                          a.ids, slot, w0, w1, lane);
  }
  if (bad) atomicAdd(&a.status[MV_PLAN_BAD_BLOCK], bad);
}

// What each wave of decode_plan_wave_kernel computes by itself, lane b
// holding sequence b (and, for a dealt plan, size bucket b).
struct WavePlan {
  bool mine, kv_ok;  // lane b < num_seqs; its kv_len is usable
  int64_t kv_raw;
  int kv, tiles, np, q, r;  // np pieces of q or q + 1 tiles (r of them q + 1)
  int ka, kb, na, nb;       // buckets of the (q + 1)- and q-tile pieces, groups in each
  int pre_a, pre_b;         // dealt: first positions of the sequence's groups in ka, kb
  int item0;                // natural order: first item
  int start, cnt;           // dealt: first position and groups of bucket `lane`
  // uniform
  int lb, part_tokens, max_parts, per_item, most_tiles, rounds, cus;
  int least_kv, bad_kv, short_table;
  int64_t num_groups, used_groups;
  bool deal, listed, fixed;
};

// Steps 1-3 of the plan for at most kWavePlanSeqs sequences, by each wave
// on its own (no barrier, no shared counts): lengths, the piece bound
// (decode_plan_kernel's rules) and the deal's positions. In the deal the
// groups are sorted by size into buckets (L - size) >> shift of 2^shift
// tiles, at most 64 (exact sizes up to L = 64 tiles, one bucket per
// lane); a group's position is its bucket's start + the groups of the
// bucket in earlier sequences + its index among its sequence's groups of
// the bucket (one scan per bucket in use, four at a time: few, the pieces
// of a batch differ little in size).
template <typename KV>
__device__ inline void wave_plan_lengths(const PlanArgs& a, WavePlan& p, int lane) {
  const KV* kvp = static_cast<const KV*>(a.kv_len);
  const int64_t bs = int64_t(1) << a.bs_log2;
  // ---- 1. lengths (kv_len outside [1, INT_MAX / 2] or beyond the table
  // row: no piece reads the sequence)
  p.mine = lane < a.num_seqs;
  p.kv_raw = p.mine ? static_cast<int64_t>(kvp[lane]) : 1;
  p.kv_ok = p.kv_raw >= 1 && p.kv_raw <= INT_MAX / 2 && (p.kv_raw + bs - 1) / bs <= a.max_blocks;
  p.kv = p.mine && p.kv_ok ? static_cast<int>(p.kv_raw) : 0;
  p.tiles = (p.kv + kTile - 1) / kTile;
}

// Steps 2-3 after wave_plan_lengths; the deal's positions only when
// `positions`.
__device__ inline void wave_plan_rest(const PlanArgs& a, WavePlan& p, int* s_used, int lane, bool positions) {
  const int hkv = a.num_kv_heads;
  s_used[lane] = 0;
  const int64_t total_tiles = wave_sum64(p.tiles);
  const int live_seqs = wave_sum(p.kv > 0);
  p.most_tiles = wave_max(p.tiles);
  p.least_kv =
      wave_min(p.mine ? static_cast<int>(vmax<int64_t>(vmin<int64_t>(p.kv_raw, INT_MAX), INT_MIN)) : INT_MAX);
  p.bad_kv = wave_sum(p.mine && p.kv_raw < 1);
  p.short_table = wave_sum(p.mine && p.kv_raw >= 1 && !p.kv_ok);
  const int64_t units = static_cast<int64_t>(live_seqs) * hkv;

  // ---- 2. piece bound L (tiles)
  const PieceRules rules =
      piece_rules(a.groups_per_cu, a.cu_count, a.bs_log2, units, total_tiles, p.most_tiles, hkv);
  const bool narrow = static_cast<int64_t>(kWavePlanSeqs) * p.most_tiles < (int64_t(1) << 30);
  const int tiles = p.tiles;
  auto groups_at = [&](int l) -> int64_t {
    const int n = static_cast<int>(static_cast<uint32_t>(tiles + l - 1) / static_cast<uint32_t>(l));
    return (narrow ? static_cast<int64_t>(wave_sum(n)) : wave_sum64(n)) * hkv;
  };
  p.lb = pick_piece_bound(rules, units, total_tiles, hkv, groups_at, p.num_groups);
  if (p.num_groups < 0) p.num_groups = groups_at(p.lb);
  p.part_tokens = p.lb * kTile;
  p.np = static_cast<int>(static_cast<uint32_t>(p.tiles + p.lb - 1) / static_cast<uint32_t>(p.lb));
  p.max_parts = wave_max(p.np);

  // ---- what the entries and id lists hold (as in decode_plan_kernel)
  p.deal = p.num_groups <= kDealMax && p.num_groups <= rules.target && a.cu_count > 0;
  p.used_groups = vmin<int64_t>(p.num_groups, a.work_cap);
  p.fixed = a.fixed_part_tokens > 0;
  p.per_item = ids_per_item(p.fixed ? a.fixed_part_tokens : p.part_tokens, a.bs_log2);
  const int64_t n_ids = p.used_groups * p.per_item;
  p.listed = p.used_groups == p.num_groups && n_ids <= a.ids_cap && n_ids <= INT_MAX &&
             (!p.fixed || p.part_tokens <= a.fixed_part_tokens);
  p.cus = vmax(1, a.cu_count);
  p.rounds = static_cast<int>(div_nonneg(p.num_groups + p.cus - 1, p.cus));

  // ---- 3. sizes, buckets, positions
  p.q = p.np > 0 ? p.tiles / p.np : 0;
  p.r = p.np > 0 ? p.tiles - p.q * p.np : 0;
  int shift = 0;
  while (((p.lb - 1) >> shift) >= 64) ++shift;
  p.kb = p.np > 0 ? (p.lb - p.q) >> shift : 0;
  p.ka = p.r > 0 ? (p.lb - p.q - 1) >> shift : p.kb;
  p.na = p.ka == p.kb ? p.np * hkv : p.r * hkv;
  p.nb = p.ka == p.kb ? 0 : (p.np - p.r) * hkv;
  p.pre_a = p.pre_b = p.item0 = p.start = p.cnt = 0;
  if (!positions) return;
  if (p.listed && p.deal) {
    // the buckets in use (flags in LDS, this wave's own copy), then in
    // ascending order, four at a time (independent scans): the groups of
    // bucket k in earlier sequences, its total and its start
    if (p.na > 0) s_used[p.ka] = 1;
    if (p.nb > 0) s_used[p.kb] = 1;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's own LDS stores
    __builtin_amdgcn_wave_barrier();
    uint64_t used = __builtin_amdgcn_ballot_w64(s_used[lane] != 0);
    int run = 0;  // positions taken by the buckets before
    while (used != 0) {
      int k[4], c[4], incl[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        k[u] = used != 0 ? __builtin_ctzll(used) : 64;
        used &= used - 1;
        c[u] = (p.ka == k[u] ? p.na : 0) + (p.kb == k[u] ? p.nb : 0);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) incl[u] = wave_scan_sum(c[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int before = incl[u] - c[u] + run;
        if (p.ka == k[u]) p.pre_a = before;
        if (p.kb == k[u]) p.pre_b = before;
        const int total = __builtin_amdgcn_readlane(incl[u], 63);
        if (lane == k[u]) {
          p.start = run;
          p.cnt = total;
        }
        run += total;
      }
    }
  } else if (p.listed) {
    p.item0 = wave_scan_sum(p.np) - p.np;  // sums at most num_groups <= INT_MAX / 4 (listed)
  }
}

// First tile, token range and whether piece j of a sequence of np pieces
// (q or q + 1 tiles, r of them q + 1) has q + 1 tiles, with bb = the
// (q + 1)-tile pieces before it, floor(j r / np).
struct PieceSpan {
  int bb, tok0, tok1;
  bool big;
};
__device__ inline PieceSpan piece_span(int kv, int np, int q, int r, int j, bool wide) {
  PieceSpan ps;
  int rem;
  if (!wide) {
    const uint32_t jr = static_cast<uint32_t>(j) * static_cast<uint32_t>(r);
    ps.bb = static_cast<int>(jr / static_cast<uint32_t>(np));
    rem = static_cast<int>(jr - static_cast<uint32_t>(ps.bb) * static_cast<uint32_t>(np));
  } else {
    const int64_t jr = static_cast<int64_t>(j) * r;
    ps.bb = static_cast<int>(jr / np);
    rem = static_cast<int>(jr - static_cast<int64_t>(ps.bb) * np);
  }
  ps.big = rem + r >= np;
  const int t0 = j * q + ps.bb;
  ps.tok0 = t0 * kTile;
  ps.tok1 = vmin(kv, (t0 + q + (ps.big ? 1 : 0)) * kTile);
  return ps;
}

// The plan of a batch of at most kWavePlanSeqs sequences (decode_plan_kernel
// for larger ones): the same rules and outputs, with every step a wave
// operation (the 1024-thread group of decode_plan_kernel spends 1.0-1.4 us
// on each of its five barrier-bound phases at c2). Each wave works the
// plan out by itself (wave_plan_lengths, wave_plan_rest), so no wave
// waits for another.
//   IDS = false: one work group; its waves write the entries of pieces
//     j / rep = wave (mod waves), rep lanes per sequence, and
//     decode_ids_kernel follows with the id lists.
//   IDS = true (a table of at most kFusedTableEntries entries): work group
//     0 writes the status, zeroes the counters and marks unused slots;
//     work group 1 checks every table entry the lengths use (from the
//     lengths alone) and writes the status's bad-entry count; with CHECK,
//     work group 2 runs the fused decode step's checks (step_check_body,
//     arguments `c`: its own status words and rows, so it shares nothing
//     with the plan); wave w of the work groups g after those takes slot
//     4 (g - first) + w, finds its piece from the positions (the inverse of
//     the deal or the natural order) and writes its entry and id list. Plan,
//     ids and checks are then one launch.
template <typename KV, typename BT, bool IDS, bool CHECK>
__global__ __launch_bounds__(64 * kWavePlanWaves) void decode_plan_wave_kernel(PlanArgs a, StepCheckArgs c) {
  static_assert(IDS || !CHECK, "the step check rides on the one-launch plan");
  __shared__ int s_used[kWavePlanWaves][64];  // size buckets in use, one copy per wave
  __shared__ int64_t s_bad[kWavePlanWaves];
  constexpr int kThreads = 64 * kWavePlanWaves;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const BT* btp = static_cast<const BT*>(a.block_table);
  const int64_t bs = int64_t(1) << a.bs_log2;
  const int hkv = a.num_kv_heads;
  if constexpr (CHECK) {
    if (blockIdx.x == 2) {
      // slot and writer tables of at most kWavePlanSeqs sequences: the host
      // sizes both to pow2(max(64, 2 num_seqs)) <= 128 entries
      __shared__ uint64_t s_slot_table[2 * kWavePlanSeqs];
      __shared__ uint64_t s_writers[2 * kWavePlanSeqs];
      __shared__ uint32_t s_dup[2 * kWavePlanSeqs / 32];
      __shared__ int s_red[2], s_cnt[2];
      __shared__ unsigned long long s_pairs;
      step_check_body<KV, BT, 64 * kWavePlanWaves, kWavePlanSeqs>(c, s_slot_table, s_writers, s_dup, s_red, s_cnt,
                                                                   &s_pairs);
      return;
    }
  }
  constexpr unsigned kFirstSlotGroup = CHECK ? 3 : 2;
  WavePlan p;
  wave_plan_lengths<KV>(a, p, lane);
  // The table check counts the entries the lengths use (rows b < num_seqs,
  // entries j < ceil(kv_b / bs), kv_b = 0 for an unusable length) outside
  // the pool: rep lanes per row, lane l taking row l / rep and its entries
  // j = l % rep + rep * (wave + waves * i), kCheckBatch loads in flight at
  // a time. It needs the lengths only: with IDS work group 1 runs it and
  // writes status[MV_PLAN_BAD_BLOCK] alone; without, it runs when there
  // are no lists (decode_ids_kernel counts otherwise).
  auto table_check = [&]() __attribute__((always_inline)) -> int64_t {
    constexpr int kCheckBatch = 16;
    const int nblk = static_cast<int>((p.kv + bs - 1) / bs);
    const int rep = vmax(1, kWavePlanSeqs / a.num_seqs);
    const int row = lane / rep < a.num_seqs ? lane / rep : -1;
    const int n = __shfl(nblk, row < 0 ? 0 : row);
    const int stride = rep * kWavePlanWaves;
    const int first = lane - (lane / rep) * rep + rep * wave;
    const BT* src = btp + static_cast<int64_t>(row < 0 ? 0 : row) * a.bt_stride;
    const int most = wave_max(row >= 0 ? n : 0);
    int64_t bad = 0;
    for (int j0 = first; j0 - first < most; j0 += kCheckBatch * stride) {  // uniform trips
      int64_t blk[kCheckBatch];
#pragma unroll
      for (int u = 0; u < kCheckBatch; ++u) {
        const int j = j0 + u * stride;
        blk[u] = row >= 0 && j < n ? static_cast<int64_t>(src[j]) : 0;
      }
#pragma unroll
      for (int u = 0; u < kCheckBatch; ++u) bad += blk[u] < 0 || blk[u] >= a.num_blocks;
    }
    bad = wave_sum64(bad);
    if (lane == 0) s_bad[wave] = bad;
    __syncthreads();
    bad = 0;
#pragma unroll
    for (int w = 0; w < kWavePlanWaves; ++w) bad += s_bad[w];
    return bad;
  };
  if (IDS && blockIdx.x == 1) {
    const int64_t bad = a.num_seqs > 0 ? table_check() : 0;
    if (threadIdx.x == 0) a.status[MV_PLAN_BAD_BLOCK] = static_cast<int32_t>(vmin<int64_t>(bad, INT_MAX));
    return;
  }
  wave_plan_rest(a, p, s_used[wave], lane, !(IDS && blockIdx.x == 0));
  const bool wide = p.most_tiles >= (1 << 16);  // j * r may exceed 32 bits

  if (IDS && blockIdx.x >= kFirstSlotGroup) {
    // ---- one slot per wave: its piece, entry and id list
    const int64_t slot = static_cast<int64_t>(blockIdx.x - kFirstSlotGroup) * kWavePlanWaves + wave;
    if (!p.listed || slot >= p.num_groups || slot >= a.work_cap) return;
    int b, j, h;
    if (p.deal) {
      const int s32 = static_cast<int>(slot);
      const int rd = static_cast<int>(static_cast<uint32_t>(s32) / static_cast<uint32_t>(p.cus));
      const int cs = s32 - rd * p.cus;
      const int pos = rd * p.cus + (((p.rounds - 1 - rd) & 1) == 0 ? cs : p.cus - 1 - cs);
      // bucket k holding pos (lane = bucket), then the sequence whose
      // groups of k hold it (lane = sequence)
      const int k = __builtin_ctzll(__builtin_amdgcn_ballot_w64(p.start <= pos && pos < p.start + p.cnt));
      const bool in_a = p.ka == k && p.pre_a <= pos && pos < p.pre_a + p.na;
      const bool in_b = p.kb == k && p.pre_b <= pos && pos < p.pre_b + p.nb;
      b = __builtin_ctzll(__builtin_amdgcn_ballot_w64(in_a || in_b));
      const bool big_b = __builtin_amdgcn_ballot_w64(in_a) != 0;  // in the (q + 1)-tile bucket
      const int idx = pos - __builtin_amdgcn_readlane(big_b ? p.pre_a : p.pre_b, b);
      const int np = __builtin_amdgcn_readlane(p.np, b), r = __builtin_amdgcn_readlane(p.r, b);
      const bool same = __builtin_amdgcn_readlane(p.ka, b) == __builtin_amdgcn_readlane(p.kb, b);
      const int i = idx / hkv;
      h = idx - i * hkv;
      // the i-th piece of b in its bucket: all pieces when both sizes share
      // it; else the i-th (q + 1)-tile piece, ceil((i + 1) np / r) - 1, or
      // the i-th q-tile piece, floor(i np / (np - r))
      if (same) j = i;
      else if (big_b) j = static_cast<int>(div_nonneg(static_cast<int64_t>(i + 1) * np + r - 1, r)) - 1;
      else j = static_cast<int>(div_nonneg(static_cast<int64_t>(i) * np, np - r));
    } else {
      const int item = static_cast<int>(slot / hkv);
      h = static_cast<int>(slot - static_cast<int64_t>(item) * hkv);
      b = __builtin_ctzll(__builtin_amdgcn_ballot_w64(p.mine && p.item0 <= item && item < p.item0 + p.np));
      j = item - __builtin_amdgcn_readlane(p.item0, b);
    }
    const int kv = __builtin_amdgcn_readlane(p.kv, b), np = __builtin_amdgcn_readlane(p.np, b);
    const PieceSpan ps = piece_span(kv, np, __builtin_amdgcn_readlane(p.q, b), __builtin_amdgcn_readlane(p.r, b),
                                    j, wide);
    const int4 w0 = make_int4(b, h, j, np);
    const int4 w1 = make_int4(ps.tok0, ps.tok1, 0, 0);
    if (lane == 0) {
      int4* w = reinterpret_cast<int4*>(a.work + 8 * slot);
      w[0] = w0;
      w[1] = w1;
    }
    write_slot_ids(btp, a.bt_stride, a.num_seqs, a.max_blocks, a.num_blocks, a.bs_log2, p.per_item, a.ids, slot,
                   w0, w1, lane);
    return;
  }

  if (!IDS && p.listed && a.num_seqs > 0) {
    // ---- 4. entries: rep lanes per sequence, lane l taking sequence l /
    // rep and its pieces j = l % rep + rep * (wave + waves * i)
    const int rep = vmax(1, kWavePlanSeqs / a.num_seqs);
    const int sb = lane / rep, m = lane - sb * rep;
    const bool act = sb < a.num_seqs;
    const int src = act ? sb : 0;
    const int kv_s = __shfl(p.kv, src), np_s = __shfl(p.np, src), q_s = __shfl(p.q, src), r_s = __shfl(p.r, src);
    const int ka_s = __shfl(p.ka, src), kb_s = __shfl(p.kb, src);
    const int pa_s = __shfl(p.pre_a, src), pb_s = __shfl(p.pre_b, src), item0_s = __shfl(p.item0, src);
    const int cus = p.cus;
    const int stride = rep * kWavePlanWaves;
    const int trips = (p.max_parts + stride - 1) / stride;
    for (int it = 0; it < trips; ++it) {  // wave-uniform trip count
      const int j = m + rep * (wave + kWavePlanWaves * it);
      if (!act || j >= np_s) continue;
      const PieceSpan ps = piece_span(kv_s, np_s, q_s, r_s, j, wide);
      // the kv heads' groups of piece j take consecutive positions
      const int pos0 = ka_s == kb_s ? pa_s + j * hkv : ps.big ? pa_s + ps.bb * hkv : pb_s + (j - ps.bb) * hkv;
      int rd = p.deal ? static_cast<int>(static_cast<uint32_t>(pos0) / static_cast<uint32_t>(cus)) : 0;
      int c = pos0 - rd * cus;
      for (int h = 0; h < hkv; ++h, ++c) {
        int64_t slot;
        if (p.deal) {
          if (c == cus) {
            ++rd;
            c = 0;
          }
          const bool forward = ((p.rounds - 1 - rd) & 1) == 0;
          slot = static_cast<int64_t>(rd) * cus + (forward ? c : cus - 1 - c);
        } else {
          slot = static_cast<int64_t>(item0_s + j) * hkv + h;
        }
        if (slot < a.work_cap) {
          int4* w = reinterpret_cast<int4*>(a.work + 8 * slot);
          w[0] = make_int4(sb, h, j, np_s);
          w[1] = make_int4(ps.tok0, ps.tok1, 0, 0);
        }
      }
    }
  }

  // ---- 5. unused slots (a launch of fixed size, or lists that do not
  // fit: then every slot), the merge counters, the table check without
  // lists (IDS: work group 1) and the status
  if (p.fixed || !p.listed) {
    for (int64_t slot = (p.listed ? p.used_groups : 0) + threadIdx.x; slot < a.work_cap; slot += kThreads) {
      int4* w = reinterpret_cast<int4*>(a.work + 8 * slot);
      w[0] = make_int4(-1, 0, 0, 0);
      w[1] = make_int4(0, 0, 0, 0);
    }
  }
  for (int64_t i = threadIdx.x; i < static_cast<int64_t>(a.num_seqs) * hkv; i += kThreads) a.counters[i] = 0;
  const int64_t bad = !IDS && !p.listed && a.num_seqs > 0 ? table_check() : 0;
  if (threadIdx.x == 0) {
    a.status[MV_PLAN_NUM_ITEMS] = static_cast<int32_t>(vmin<int64_t>(p.num_groups, INT_MAX));
    a.status[MV_PLAN_BAD_KV_LEN] = p.bad_kv;
    a.status[MV_PLAN_INSUFFICIENT] = p.short_table;
    if (!IDS) a.status[MV_PLAN_BAD_BLOCK] = static_cast<int32_t>(vmin<int64_t>(bad, INT_MAX));
    a.status[MV_PLAN_MAX_PARTS] = p.max_parts;
    a.status[MV_PLAN_MIN_KV_LEN] = a.num_seqs > 0 ? p.least_kv : 0;
    a.status[MV_PLAN_PARTITION_TOKENS] = p.part_tokens;
    a.status[MV_PLAN_IDS_PER_ITEM] = p.listed ? p.per_item : -1;
  }
}

// ------------------------------------------------------------- dispatch ---

// Partial O rows sized as fp32 for every dtype (the workspace size takes no
// dtype); 16-bit rows use the first half.
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

// Three tile stages instead of two for a launch of short pieces over a
// batch of few units per CU -- at least kDeepMinUnits (sequence, kv head)
// units, at least two groups per unit (the plan's two groups per CU) and
// pieces of at most kDeepPieceTokens: c2-like batches, whose waves stream
// a few tiles each, gain from the deeper prefetch (layer call 10.65-10.74
// against 10.57-10.69 us, four same-box pairs), while long pieces (c3,
// 1504 tokens: 36.0-36.2 -> 37.0-37.3 us), three groups per CU (c4: 15.8
// -> 17.1 us) and launches of a handful of groups (batches of 1-4
// sequences: +0.04 to +0.1 us) lose. Tiles over 2 KiB keep two stages.
constexpr int kDeepPieceTokens = 512;
constexpr int kDeepMinUnits = 64;

template <int DTYPE, int D, int SREQ>
int launch_decode_s(const DecodeArgs& a, int num_groups, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(num_groups);
  if (a.rope_cos) paged_decode_kernel<DTYPE, D, true, true, SREQ><<<grid, kWaves * 64, 0, s>>>(a);
  else if (a.new_k) paged_decode_kernel<DTYPE, D, true, false, SREQ><<<grid, kWaves * 64, 0, s>>>(a);
  else paged_decode_kernel<DTYPE, D, false, false, SREQ><<<grid, kWaves * 64, 0, s>>>(a);
  return check_launch("mv_paged_decode");
}

template <int DTYPE, int D>
int launch_decode(const DecodeArgs& a, int num_groups, bool deep, hipStream_t s) {
  if constexpr (Traits<DTYPE, D, 3>::kStages == 3 && MV_DECODE_STAGES == 2) {
    if (deep) return launch_decode_s<DTYPE, D, 3>(a, num_groups, s);
  }
  return launch_decode_s<DTYPE, D, MV_DECODE_STAGES>(a, num_groups, s);
}

template <int DTYPE>
int launch_decode_d(const DecodeArgs& a, int d, int num_groups, bool deep, hipStream_t s) {
  return d == 64 ? launch_decode<DTYPE, 64>(a, num_groups, deep, s)
                 : launch_decode<DTYPE, 128>(a, num_groups, deep, s);
}

// The step's new rows for the fused KV write (mv_paged_decode_write).
struct NewRows {
  const void* key;
  int64_t key_stride_tok, key_stride_head;      // elements
  const void* value;
  int64_t value_stride_tok, value_stride_head;  // elements
  const int64_t* slots;
  const void* rope_cos;  // [num_seqs][head_dim] rows, or null (no RoPE)
  const void* rope_sin;
};

// What any plan of a batch can produce (the plan kernel's own rules):
// its piece bound L never exceeds l_cap and never falls below
// min(l_cap, kWaves) (l_cap >= 31 for block sizes >= 1); its groups number
// at most the resident target when L comes from the search, else (L >= the
// fair share, or L = l_cap) at most units + total tiles / L.
struct PlanBounds {
  int64_t groups, l_cap, max_parts;
};
inline PlanBounds plan_bounds(int32_t num_seqs, int32_t max_blocks, int32_t block_size,
                              int32_t num_kv_heads, int32_t groups_per_cu, int32_t cu_count) {
  const int bs_log2 = ilog2_exact(block_size);
  const int64_t l_cap = std::max<int64_t>(
      1, std::min<int64_t>(INT_MAX / 32, (static_cast<int64_t>(kIdCap - 1) << bs_log2) / kTile));
  const int64_t max_tiles = (static_cast<int64_t>(max_blocks) * block_size + kTile - 1) / kTile;
  const int64_t max_parts =
      std::max<int64_t>(1, std::min<int64_t>(kMaxParts, (max_tiles + kWaves - 1) / kWaves));
  const int64_t units = static_cast<int64_t>(num_kv_heads) * num_seqs;
  // at least the plan's resident target (kFewUnitsPerCU per CU when its
  // live units fit the CUs, else up to kManyUnitsPerCU)
  const int gpc = std::max(1, groups_per_cu);
  const int64_t target =
      static_cast<int64_t>(units <= cu_count ? std::min(kFewUnitsPerCU, gpc)
                                             : std::max(kFewUnitsPerCU, std::min(kManyUnitsPerCU, gpc))) *
      std::max(1, cu_count);
  const int64_t by_fair = units + std::max<int64_t>(target, (units * max_tiles + l_cap - 1) / l_cap);
  return PlanBounds{std::min<int64_t>(by_fair, units * max_parts), l_cap, max_parts};
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

extern "C" int mv_decode_graph_bounds(int32_t num_seqs, int32_t max_blocks, int32_t block_size,
                                      int32_t num_kv_heads, int32_t groups_per_cu,
                                      int32_t cu_count, int64_t* out) {
  using namespace mv;
  if (!out) return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_graph_bounds: null out");
  if (num_seqs <= 0 || max_blocks <= 0 || num_kv_heads <= 0 || cu_count <= 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_graph_bounds: bad sizes");
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "mv_decode_graph_bounds: block_size %d is not a power of 2",
                block_size);
  const mv::PlanBounds pb = mv::plan_bounds(num_seqs, max_blocks, block_size, num_kv_heads,
                                            groups_per_cu, cu_count);
  if (pb.groups > INT_MAX / 8)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_graph_bounds: batch too large");
  out[0] = pb.groups;
  out[1] = pb.l_cap * kTile;
  out[2] = pb.max_parts;
  return MV_OK;
}

extern "C" int64_t mv_decode_block_ids_capacity(int32_t num_seqs, int32_t max_blocks,
                                                int32_t num_kv_heads, int64_t work_capacity) {
  if (num_seqs < 0 || max_blocks < 0 || num_kv_heads < 0 || work_capacity < 0) return 0;
  // Sequence b (T_b tiles) is cut into np_b = ceil(T_b / L) pieces of at
  // most P = 16 L tokens, and ids_per_item <= ceil(P / bs) + 4. np_b * P <
  // 16 T_b + P <= kv_b + 15 + P, so np_b * ids_per_item <= (kv_b + 15 + P)
  // / bs + 5 np_b <= max_blocks + 15 + kIdCap + 5 np_b (P <= (kIdCap - 1)
  // * bs); per kv head.
  return static_cast<int64_t>(num_kv_heads) * num_seqs * (max_blocks + mv::kIdCap + 16) +
         5 * work_capacity;
}

extern "C" size_t mv_paged_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                  int32_t head_dim, int32_t max_partitions) {
  if (max_partitions <= 1 || num_seqs <= 0 || num_q_heads <= 0 || head_dim <= 0) return 0;
  const size_t o = mv::ws_o_bytes(num_seqs, num_q_heads, head_dim, max_partitions);
  const size_t ml = static_cast<size_t>(num_seqs) * num_q_heads * max_partitions * sizeof(float2);
  return ((o + 255) / 256) * 256 + ml;
}

namespace mv {
namespace {

// Validates mv_decode_plan's arguments and fills `a`.
int plan_prepare(const char* who, const void* kv_len, const void* block_table, int64_t bt_stride,
                 int32_t num_seqs, int32_t max_blocks, int32_t block_size, int64_t num_blocks,
                 int32_t num_kv_heads, int32_t groups_per_cu, int32_t cu_count,
                 int32_t fixed_partition_tokens, int32_t* work_items, int64_t work_capacity,
                 int32_t* block_ids, int64_t block_ids_capacity, int32_t* counters, int32_t* status,
                 PlanArgs* a) {
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "%s: null status", who);
  if (num_seqs < 0 || max_blocks < 0 || work_capacity < 0 || block_ids_capacity < 0 ||
      num_blocks < 0 || num_kv_heads <= 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: bad sizes", who);
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "%s: block_size %d is not a power of 2", who, block_size);
  if (num_seqs > 0 && (!kv_len || !counters || (max_blocks > 0 && !block_table)))
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: null pointer", who);
  if ((work_capacity > 0 && !work_items) || (block_ids_capacity > 0 && !block_ids))
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: null work list", who);
  const int64_t ids_need =
      mv_decode_block_ids_capacity(num_seqs, max_blocks, num_kv_heads, work_capacity);
  if (block_ids_capacity < ids_need)
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: block_ids capacity %lld < %lld", who,
                static_cast<long long>(block_ids_capacity), static_cast<long long>(ids_need));
  a->kv_len = kv_len;
  a->block_table = block_table;
  a->bt_stride = bt_stride;
  a->num_seqs = num_seqs;
  a->max_blocks = max_blocks;
  a->bs_log2 = ilog2_exact(block_size);
  a->num_kv_heads = num_kv_heads;
  a->groups_per_cu = groups_per_cu;
  a->cu_count = cu_count;
  a->fixed_part_tokens = fixed_partition_tokens;
  a->num_blocks = num_blocks;
  a->work = work_items;
  a->work_cap = work_capacity;
  a->ids = block_ids;
  a->ids_cap = block_ids_capacity;
  a->counters = counters;
  a->status = status;
  return MV_OK;
}

template <typename KV, typename BT, bool IDS, bool CHECK>
void launch_wave_plan(unsigned grid, const PlanArgs& a, const StepCheckArgs& c, hipStream_t s) {
  decode_plan_wave_kernel<KV, BT, IDS, CHECK><<<grid, 64 * kWavePlanWaves, 0, s>>>(a, c);
}

template <bool IDS, bool CHECK>
void launch_wave_plan(unsigned grid, int32_t kv_len_is_i64, int32_t bt_is_i64, const PlanArgs& a,
                      const StepCheckArgs& c, hipStream_t s) {
  if (kv_len_is_i64) {
    if (bt_is_i64) launch_wave_plan<int64_t, int64_t, IDS, CHECK>(grid, a, c, s);
    else launch_wave_plan<int64_t, int32_t, IDS, CHECK>(grid, a, c, s);
  } else {
    if (bt_is_i64) launch_wave_plan<int32_t, int64_t, IDS, CHECK>(grid, a, c, s);
    else launch_wave_plan<int32_t, int32_t, IDS, CHECK>(grid, a, c, s);
  }
}

// Enqueues the plan of `a` and its id lists; with `chk` (fused decode step
// checks, arguments validated) the step check and its shared-read scan too.
// Up to kWavePlanSeqs sequences over a table of at most kFusedTableEntries
// entries the plan, the id lists and the step check are one launch.
int plan_enqueue(const char* who, const PlanArgs& a, int32_t kv_len_is_i64, int32_t bt_is_i64,
                 int32_t block_size, const StepCheckArgs* chk, hipStream_t s) {
  // slots the plan can fill (the same bound as a launch of fixed size)
  const int64_t slots = std::min<int64_t>(
      a.work_cap, plan_bounds(a.num_seqs, a.max_blocks, block_size, a.num_kv_heads, a.groups_per_cu, a.cu_count)
                      .groups);
  const bool wave_plan = a.num_seqs <= kWavePlanSeqs;
  // plan and id lists in one launch: a small table (work group 1 checks all
  // of it) and lists to write; one wave per slot after the first groups
  const bool fused = wave_plan && a.num_seqs > 0 && a.ids_cap > 0 &&
                     static_cast<int64_t>(a.num_seqs) * a.max_blocks <= kFusedTableEntries &&
                     slots <= kFusedSlots;
  StepCheckArgs none{};
  if (fused) {
    // the step check's work group holds tables of pow2(max(64, 2 num_seqs))
    // <= 2 kWavePlanSeqs entries
    const bool with_check = chk && chk->slot_hmask < 2 * kWavePlanSeqs && chk->writer_hmask < 2 * kWavePlanSeqs;
    const unsigned first = with_check ? 3 : 2;
    const unsigned grid = first + static_cast<unsigned>((slots + kWavePlanWaves - 1) / kWavePlanWaves);
    if (with_check) launch_wave_plan<true, true>(grid, kv_len_is_i64, bt_is_i64, a, *chk, s);
    else launch_wave_plan<true, false>(grid, kv_len_is_i64, bt_is_i64, a, none, s);
    if (const int rc = check_launch(who)) return rc;
    if (chk && !with_check) step_check_launch(*chk, bt_is_i64, kv_len_is_i64, s);
    else if (chk) step_check_scan(*chk, bt_is_i64, kv_len_is_i64, s);
    return check_launch(who);
  }
  if (wave_plan) {
    launch_wave_plan<false, false>(1, kv_len_is_i64, bt_is_i64, a, none, s);
  } else if (kv_len_is_i64) {
    if (bt_is_i64) decode_plan_kernel<int64_t, int64_t><<<1, kPlanThreads, 0, s>>>(a);
    else decode_plan_kernel<int64_t, int32_t><<<1, kPlanThreads, 0, s>>>(a);
  } else {
    if (bt_is_i64) decode_plan_kernel<int32_t, int64_t><<<1, kPlanThreads, 0, s>>>(a);
    else decode_plan_kernel<int32_t, int32_t><<<1, kPlanThreads, 0, s>>>(a);
  }
  if (const int rc = check_launch(who)) return rc;
  if (a.num_seqs > 0 && a.ids_cap > 0) {
    IdsArgs d;
    d.block_table = a.block_table;
    d.bt_stride = a.bt_stride;
    d.num_seqs = a.num_seqs;
    d.max_blocks = a.max_blocks;
    d.work = a.work;
    d.work_cap = a.work_cap;
    d.ids = a.ids;
    d.status = a.status;
    d.num_blocks = a.num_blocks;
    d.bs_log2 = a.bs_log2;
    // one wave per slot the plan can fill, in one pass up to 4096 work groups
    constexpr int64_t kSlotsPerGroup = kIdsThreads / 64;
    const int grid = static_cast<int>(std::min<int64_t>(
        4096, std::max<int64_t>(1, (slots + kSlotsPerGroup - 1) / kSlotsPerGroup)));
    if (bt_is_i64) decode_ids_kernel<int64_t><<<grid, kIdsThreads, 0, s>>>(d);
    else decode_ids_kernel<int32_t><<<grid, kIdsThreads, 0, s>>>(d);
  }
  if (chk) step_check_launch(*chk, bt_is_i64, kv_len_is_i64, s);
  return check_launch(who);
}

}  // namespace
}  // namespace mv

extern "C" int mv_decode_plan(const void* kv_len, int32_t kv_len_is_i64, const void* block_table,
                              int32_t bt_is_i64, int64_t bt_stride, int32_t num_seqs,
                              int32_t max_blocks, int32_t block_size, int64_t num_blocks,
                              int32_t num_kv_heads, int32_t groups_per_cu,
                              int32_t cu_count, int32_t fixed_partition_tokens,
                              int32_t* work_items, int64_t work_capacity,
                              int32_t* block_ids,
                              int64_t block_ids_capacity, int32_t* counters, int32_t* status,
                              void* stream) {
  using namespace mv;
  PlanArgs a;
  if (const int rc = plan_prepare("mv_decode_plan", kv_len, block_table, bt_stride, num_seqs, max_blocks,
                                  block_size, num_blocks, num_kv_heads, groups_per_cu, cu_count,
                                  fixed_partition_tokens, work_items, work_capacity, block_ids,
                                  block_ids_capacity, counters, status, &a))
    return rc;
  return plan_enqueue("mv_decode_plan", a, kv_len_is_i64, bt_is_i64, block_size, nullptr,
                      static_cast<hipStream_t>(stream));
}

extern "C" int mv_decode_plan_step_check(
    const void* kv_len, int32_t kv_len_is_i64, const void* block_table, int32_t bt_is_i64, int64_t bt_stride,
    int32_t num_seqs, int32_t max_blocks, int32_t block_size, int64_t num_blocks, int32_t num_kv_heads,
    int32_t groups_per_cu, int32_t cu_count, int32_t fixed_partition_tokens, int32_t* work_items,
    int64_t work_capacity, int32_t* block_ids, int64_t block_ids_capacity, int32_t* counters, int32_t* status,
    const int64_t* slot_mapping, const int64_t* positions, const void* cos_table, const void* sin_table,
    int64_t table_stride, int64_t max_positions, int32_t head_dim, int32_t dtype, void* cos_rows,
    void* sin_rows, int32_t* step_status, void* check_workspace, size_t check_workspace_bytes, void* stream) {
  using namespace mv;
  constexpr const char* who = "mv_decode_plan_step_check";
  PlanArgs a;
  if (const int rc = plan_prepare(who, kv_len, block_table, bt_stride, num_seqs, max_blocks, block_size,
                                  num_blocks, num_kv_heads, groups_per_cu, cu_count, fixed_partition_tokens,
                                  work_items, work_capacity, block_ids, block_ids_capacity, counters, status, &a))
    return rc;
  StepCheckArgs c;
  if (const int rc = step_check_prepare(who, slot_mapping, block_table, bt_stride, kv_len, num_seqs, max_blocks,
                                        block_size, num_blocks, positions, cos_table, sin_table, table_stride,
                                        max_positions, head_dim, dtype, cos_rows, sin_rows, step_status,
                                        check_workspace, check_workspace_bytes, &c))
    return rc;
  return plan_enqueue(who, a, kv_len_is_i64, bt_is_i64, block_size, &c, static_cast<hipStream_t>(stream));
}

namespace mv {
int decode_launch(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                               const void* key_cache, const void* value_cache,
                               const int32_t* work_items, const int32_t* block_ids,
                               int64_t block_ids_capacity, int32_t num_work_groups,
                               int32_t partition_tokens, int32_t max_partitions, int32_t* counters,
                               void* out, int64_t out_stride_tok, int64_t out_stride_head,
                               float scale, int32_t num_seqs, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               int64_t num_blocks, int32_t dtype, void* workspace,
                               size_t workspace_bytes, const NewRows* nr, void* stream) {
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
  if (num_seqs < 0 || num_work_groups < 0 || num_blocks <= 0 || max_partitions < 0 ||
      block_ids_capacity < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: bad sizes");
  if (partition_tokens <= 0 || partition_tokens % kTile)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_paged_decode: partition_tokens %d is not a positive multiple of %d",
                partition_tokens, kTile);
  if ((static_cast<int64_t>(partition_tokens) + block_size - 1) / block_size + 1 > kIdCap)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_paged_decode: partition_tokens %d spans more than %d blocks of %d tokens",
                partition_tokens, kIdCap - 1, block_size);
  if (num_seqs == 0 || num_work_groups == 0) return MV_OK;
  if (!query || !key_cache || !value_cache || !work_items || !block_ids || !out)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: null pointer");
  const int bs_log2 = ilog2_exact(block_size);
  const int per_item = ids_per_item(partition_tokens, bs_log2);
  if (static_cast<int64_t>(num_work_groups) * per_item > block_ids_capacity)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_paged_decode: %d work groups x %d block ids exceed capacity %lld",
                num_work_groups, per_item, static_cast<long long>(block_ids_capacity));
  // 16-byte copies of q rows, cache rows and block-id lists.
  if ((reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(key_cache) |
       reinterpret_cast<uintptr_t>(value_cache) | reinterpret_cast<uintptr_t>(block_ids) |
       reinterpret_cast<uintptr_t>(work_items)) % 16 ||
      (q_stride_tok * eb) % 16 || (q_stride_head * eb) % 16)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_paged_decode: query/cache rows or plan arrays not 16-byte aligned");
  if (max_partitions > 0 &&
      num_work_groups > static_cast<int64_t>(max_partitions) * num_seqs * num_kv_heads)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: work list larger than the plan allows");

  DecodeArgs a;
  a.q = query;
  a.q_stride_tok = q_stride_tok;
  a.q_stride_head = q_stride_head;
  a.k_cache = static_cast<const char*>(key_cache);
  a.v_cache = static_cast<const char*>(value_cache);
  a.work = work_items;
  a.block_ids = block_ids;
  a.ids_per_item = per_item;
  a.counters = counters;
  a.out = out;
  a.out_stride_tok = out_stride_tok;
  a.out_stride_head = out_stride_head;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.inv_scale_log2 = 1.f / a.scale_log2;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.n_rep = n_rep;
  a.bs_log2 = bs_log2;
  a.max_parts = max_partitions;
  a.num_blocks_u32 = static_cast<uint32_t>(std::min<int64_t>(num_blocks, int64_t(1) << 31));
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
  a.new_k = nullptr;
  a.new_v = nullptr;
  a.nk_st = a.nk_sh = a.nv_st = a.nv_sh = 0;
  a.slots = nullptr;
  a.total_slots = num_blocks * block_size;
  a.rope_cos = nullptr;
  a.rope_sin = nullptr;
  if (nr) {
    if (!nr->key || !nr->value || !nr->slots)
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode_write: null new rows or slots");
    if ((reinterpret_cast<uintptr_t>(nr->key) | reinterpret_cast<uintptr_t>(nr->value)) % 16 ||
        ((nr->key_stride_tok | nr->key_stride_head | nr->value_stride_tok |
          nr->value_stride_head) * eb) % 16)
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode_write: new rows not 16-byte aligned");
    a.new_k = static_cast<const char*>(nr->key);
    a.new_v = static_cast<const char*>(nr->value);
    a.nk_st = nr->key_stride_tok * eb;
    a.nk_sh = nr->key_stride_head * eb;
    a.nv_st = nr->value_stride_tok * eb;
    a.nv_sh = nr->value_stride_head * eb;
    a.slots = nr->slots;
    if ((nr->rope_cos == nullptr) != (nr->rope_sin == nullptr))
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode_write: give both RoPE rows or neither");
    if ((reinterpret_cast<uintptr_t>(nr->rope_cos) | reinterpret_cast<uintptr_t>(nr->rope_sin)) % 16)
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode_write: RoPE rows not 16-byte aligned");
    a.rope_cos = static_cast<const char*>(nr->rope_cos);
    a.rope_sin = static_cast<const char*>(nr->rope_sin);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t units = static_cast<int64_t>(num_seqs) * num_kv_heads;
  const bool deep = partition_tokens <= kDeepPieceTokens && units >= kDeepMinUnits &&
                    static_cast<int64_t>(num_work_groups) >= 2 * units;
  switch (dtype) {
    case MV_DTYPE_F32: return launch_decode_d<MV_DTYPE_F32>(a, head_dim, num_work_groups, deep, s);
    case MV_DTYPE_F16: return launch_decode_d<MV_DTYPE_F16>(a, head_dim, num_work_groups, deep, s);
    default: return launch_decode_d<MV_DTYPE_BF16>(a, head_dim, num_work_groups, deep, s);
  }
}
}  // namespace mv

extern "C" int mv_paged_decode(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                               const void* key_cache, const void* value_cache,
                               const int32_t* work_items, const int32_t* block_ids,
                               int64_t block_ids_capacity, int32_t num_work_groups,
                               int32_t partition_tokens, int32_t max_partitions, int32_t* counters,
                               void* out, int64_t out_stride_tok, int64_t out_stride_head,
                               float scale, int32_t num_seqs, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               int64_t num_blocks, int32_t dtype, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return mv::decode_launch(query, q_stride_tok, q_stride_head, key_cache, value_cache, work_items,
                           block_ids, block_ids_capacity, num_work_groups, partition_tokens,
                           max_partitions, counters, out, out_stride_tok, out_stride_head, scale,
                           num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
                           dtype, workspace, workspace_bytes, nullptr, stream);
}

// ---------------------------------------------------- no-allocation decode ---
// mv_paged_decode for callers that cannot allocate (graph capture, serving
// loops that forbid it): the partials of the split-K merge live in this
// file-scope array instead of a caller's workspace. Every GPU the library
// runs on holds one copy (MV_DECODE_SCRATCH_BYTES) until the process ends;
// all calls on that GPU share it, so calls that overlap on one GPU race.
// The merge writes every partial it reads in the same launch, so nothing in
// it has to start at zero.
static __device__ __align__(256) char scratch[MV_DECODE_SCRATCH_BYTES];

namespace {
constexpr int kScratchMaxDevices = 256;
std::atomic<void*> g_scratch_ptr[kScratchMaxDevices];
std::mutex g_scratch_mutex;

// The device address of `scratch` on the current device, looked up once per
// device with that device current (hipGetSymbolAddress): the array's name in
// host code is only a host-side stand-in.
int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return mv::fail(MV_ERR_HIP, "mv_paged_decode_noalloc: hipGetDevice: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kScratchMaxDevices)
    return mv::fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode_noalloc: device %d out of range", dev);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess || !p)
        return mv::fail(MV_ERR_HIP, "mv_paged_decode_noalloc: hipGetSymbolAddress: %s",
                        hipGetErrorString(err));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return MV_OK;
}
}  // namespace

extern "C" int mv_paged_decode_noalloc(const void* query, int64_t q_stride_tok,
                                       int64_t q_stride_head, const void* key_cache,
                                       const void* value_cache, const int32_t* work_items,
                                       const int32_t* block_ids, int64_t block_ids_capacity,
                                       int32_t num_work_groups, int32_t partition_tokens,
                                       int32_t max_partitions, int32_t* counters, void* out,
                                       int64_t out_stride_tok, int64_t out_stride_head,
                                       float scale, int32_t num_seqs, int32_t num_q_heads,
                                       int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                       int64_t num_blocks, int32_t dtype, void* stream) {
  if (num_seqs < 0 || num_q_heads < 0 || head_dim < 0 || max_partitions < 0)
    return mv::fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode_noalloc: bad sizes");
  const size_t need =
      mv_paged_decode_workspace_bytes(num_seqs, num_q_heads, head_dim, max_partitions);
  if (need > static_cast<size_t>(MV_DECODE_SCRATCH_BYTES))
    return mv::fail(MV_ERR_INVALID_ARGUMENT,
                    "mv_paged_decode_noalloc: the merge needs %zu bytes of scratch, more than "
                    "its %d-byte static buffer (%d sequences x %d query heads x %d partitions); "
                    "use mv_paged_decode with a workspace",
                    need, MV_DECODE_SCRATCH_BYTES, num_seqs, num_q_heads, max_partitions);
  int stream_dev = -1, cur = -1;
  if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_dev) != hipSuccess ||
      hipGetDevice(&cur) != hipSuccess || stream_dev != cur)
    return mv::fail(MV_ERR_INVALID_ARGUMENT,
                    "mv_paged_decode_noalloc: the stream must belong to the current device");
  void* ws = nullptr;
  if (const int rc = scratch_on_current_device(&ws)) return rc;
  return mv::decode_launch(query, q_stride_tok, q_stride_head, key_cache, value_cache, work_items,
                           block_ids, block_ids_capacity, num_work_groups, partition_tokens,
                           max_partitions, counters, out, out_stride_tok, out_stride_head, scale,
                           num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
                           dtype, ws, MV_DECODE_SCRATCH_BYTES, nullptr, stream);
}

extern "C" int mv_paged_decode_write(
    const void* query, int64_t q_stride_tok, int64_t q_stride_head, const void* new_key,
    int64_t nk_stride_tok, int64_t nk_stride_head, const void* new_value, int64_t nv_stride_tok,
    int64_t nv_stride_head, const int64_t* slot_mapping, const void* rope_cos_rows,
    const void* rope_sin_rows, void* key_cache, void* value_cache,
    const int32_t* work_items, const int32_t* block_ids, int64_t block_ids_capacity,
    int32_t num_work_groups, int32_t partition_tokens, int32_t max_partitions, int32_t* counters,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, float scale, int32_t num_seqs,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int64_t num_blocks, int32_t dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const mv::NewRows nr{new_key, nk_stride_tok, nk_stride_head, new_value, nv_stride_tok,
                       nv_stride_head, slot_mapping, rope_cos_rows, rope_sin_rows};
  return mv::decode_launch(query, q_stride_tok, q_stride_head, key_cache, value_cache, work_items,
                           block_ids, block_ids_capacity, num_work_groups, partition_tokens,
                           max_partitions, counters, out, out_stride_tok, out_stride_head, scale,
                           num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
                           dtype, workspace, workspace_bytes, &nr, stream);
}
