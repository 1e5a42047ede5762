// Paged prefill attention for gfx950 (MI355X), wave64 + MFMA.
//
// Math (AttentionBackendGPU.prefill_attention,
// mini_vllm/attention/paged_attention_gpu.py:577-661): for every prefill
// sequence with `cached` tokens already in the pool and a chunk of
// `q_len` new tokens,
//   keys 0 .. cached-1     from the pool (table row `seq_indices[i]`),
//   keys cached .. +q_len  from the chunk's own key / value rows,
//   out[t, hq] = softmax_j<=cached+t(scale * q[t, hq] . k_j) v_j,
// kv head hk = hq / n_rep, scale = head_dim^-1/2 -- the reference's
// gather + cat + repeat_interleave + masked SDPA, in one pass over the
// keys with no gathered copy.
//
// Work decomposition: one work group of W waves (8, or 4 for fp32 at
// head_dim 128) per (sequence, kv head, block of query tokens). A wave owns
// 16 R MFMA rows; row r is query head (h * n_rep + r % n_rep) of token
// (r / n_rep) of the wave's tpw = 16 R / n_rep tokens, so one K/V pass
// serves the whole GQA group of the work group's tokens. The waves share
// one stream of keys:
//   * a stage is 16 W T keys: wave w copies sub-tiles w, w + W, .. (T of
//     them, 16 keys of K and V each) from HBM straight to LDS
//     (global_load_lds, XOR piece swizzle as in the decode kernel), two
//     stages in flight;
//   * after one barrier per stage every wave computes its set's sub-tiles
//     for its rows: S^T = K Q^T (MFMA), per-row causal mask key <= cached +
//     token, online softmax, O += P V (MFMA, V read by transposed LDS loads);
//   * prefix keys are addressed through the sequence's block ids, staged
//     in LDS per window of kPfIdCap blocks; chunk keys through the chunk's
//     row strides (q / k / v may be views of one fused QKV output).
// 16-bit types at head_dim 64 run two sets of W/2 waves (R = 2, T = 2)
// that split every stage's sub-tiles and merge their softmax states at the
// end; the other instantiations one set (R = 1, T = 1). Waves skip
// sub-tiles that lie wholly past their rows' causal limit; the online
// softmax is updated once per stage.
//
// Key split (mv_paged_prefill_parts): when a launch has fewer (sequence, kv
// head, token block) units than the device has CUs, the host cuts a unit's
// keys into parts at stage boundaries, one work group each. A part leaves
// its rows' normalised O and (max, sum) in a workspace with device-coherent
// stores and counts itself on the unit's counter; the work group that
// completes the count folds the parts in part order (log-sum-exp) and
// writes the rows, so the result does not depend on which part finishes
// last.
#include <algorithm>
#include <climits>

#include "mv_coherent.h"
#include "mv_common.h"
#include "mv_tile.h"

namespace mv {
namespace {

constexpr int kPfIdCap = 2048;  // prefix block ids staged in LDS per window
// Key split: at most kPfMaxParts parts per unit, kPfMaxUnits units per launch
// (the workspace's counters come first, kPfCountersBytes of them).
constexpr int kPfMaxParts = 8;
constexpr int kPfMaxUnits = 16384;
constexpr int kPfCountersBytes = kPfMaxUnits * 4;
// 16-bit types: a stage keeps p = exp2(s - m) with the row's reference m
// unchanged when every row's stage sum lies in [kPfFastMin, kPfFastMax].
constexpr float kPfFastMax = 4096.f;
constexpr float kPfFastMin = 1.f / 4096.f;
// Waves per work group: 8 (twice the query rows per pass over the keys,
// and more waves to hide latency -- 39.8 us against 46.7 us with 4, two
// such groups then sharing a CU, on a 4 x (1536 + 512) bf16 step) when two
// stages of 8 sub-tiles fit the LDS, else 4 (fp32 at head_dim 128). Two
// stages: a third measured no faster.
// 16-row MFMA tiles per wave in one set of waves: one. Two with 8 waves
// (32 tokens per work group) halve the work groups: 57.6 against 38.2 us
// on that step, though 18 % faster per sequence at 16 sequences, where
// there are enough work groups; the two sets below keep 16 tokens per
// work group with two tiles per wave.
#ifndef MV_PREFILL_WAVES
#define MV_PREFILL_WAVES 8
#endif
#ifndef MV_PREFILL_ROWS
#define MV_PREFILL_ROWS 1
#endif
// 16-bit types at head_dim 64 (the Qwen2 shapes):
// * Key split inside the work group: two sets of W/2 waves hold the same
//   rows, two 16-row tiles per wave, and each set computes half of every
//   stage's sub-tiles; the sets' softmax states are merged through LDS at
//   the end. Every K/V byte staged in LDS is read by W/2 waves instead of W.
// * Two sub-tiles copied per wave, so a stage is 256 keys: half the
//   barriers, copy rounds and per-stage softmax exchanges per key.
// Together 35.8 against 38.1 us on a 4 x (1536 + 512) bf16 step; either
// alone measured no faster (38.8, 38.5 us).
#ifndef MV_PREFILL_SETS
#define MV_PREFILL_SETS 2
#endif
#ifndef MV_PREFILL_WAVE_TILES
#define MV_PREFILL_WAVE_TILES 2
#endif
// P V at head_dim 64 by one 16x16x32 MFMA per pair of sub-tiles: a
// 16x16x16 bf16 MFMA issues every 18.6 cycles and a 16x16x32 one, twice
// the work, every 16.6 (one wave, measured), so pairing halves the PV
// MFMA time (38.2 against 40.2 us on the step above).
#ifndef MV_PREFILL_PV32
#define MV_PREFILL_PV32 1
#endif
template <int DTYPE, int D>
struct PfTraits : TileGeom<DTYPE, D> {
  using G = TileGeom<DTYPE, D>;
  static constexpr int kSubBytes = 2 * G::kTileBytes;  // K and V sub-tile of one wave
  static constexpr int kStages = 2;
  static constexpr int kWaveTiles =  // sub-tiles each wave copies per stage
      DTYPE != MV_DTYPE_F32 && D == 64 ? MV_PREFILL_WAVE_TILES : 1;
  static constexpr int kWaves =
      kStages * MV_PREFILL_WAVES * kSubBytes * kWaveTiles + kPfIdCap * 4 <= 160 * 1024 ? MV_PREFILL_WAVES : 4;
  // sets of waves splitting each stage's sub-tiles (same rows in every set)
  static constexpr int kSets = DTYPE != MV_DTYPE_F32 && D == 64 && kWaves % (2 * MV_PREFILL_SETS) == 0
                                   ? MV_PREFILL_SETS : 1;
  static constexpr int kRowWaves = kWaves / kSets;      // waves with distinct rows
  static constexpr int kSetTiles = kWaves * kWaveTiles / kSets;  // sub-tiles per set and stage
  static constexpr int kRows = MV_PREFILL_ROWS * kSets;  // 16-row MFMA tiles per wave
  static constexpr int kStageTokens = kWaves * kWaveTiles * kTile;
  static constexpr int kStageBytes = kWaves * kWaveTiles * kSubBytes;
  static constexpr int kIdsOffset = kStages * kStageBytes;
  static constexpr int kLdsBytes = kIdsOffset + kPfIdCap * 4;
  static_assert(kLdsBytes <= 160 * 1024, "LDS of one work group");
  static_assert(kSetTiles % 2 == 0, "sub-tiles are paired for the 16x16x32 PV MFMA");
  // the set merge reuses the stage buffers: m, l and O of every row wave
  static constexpr int kMergeFloats = kRows * 16 * 2 + kRows * D * 16;
  static_assert(kSets == 1 || kRowWaves * kMergeFloats * 4 <= kIdsOffset, "set merge in LDS");
};

// Query tokens one work group covers: 16 kRows MFMA rows per row wave hold
// floor(16 kRows / n_rep) tokens' GQA groups.
template <int DTYPE, int D>
constexpr int pf_tokens_per_group(int n_rep) {
  using Tr = PfTraits<DTYPE, D>;
  return n_rep > 16 ? 0 : Tr::kRowWaves * (16 * Tr::kRows / n_rep);
}

struct PrefillArgs {
  const int32_t* work;   // per work group: (sequence, kv head, first token, tokens)
  const int64_t* seqs;   // per sequence: (table row, cached tokens, first chunk row, chunk tokens)
  const void* q;
  const char* k_new;
  const char* v_new;
  const char* k_cache;
  const char* v_cache;
  const void* block_table;
  void* out;
  int64_t q_st, q_sh;     // elements
  int64_t k_st, k_sh;     // bytes
  int64_t v_st, v_sh;     // bytes
  int64_t o_st, o_sh;     // elements
  int64_t bt_stride;      // elements
  float scale_log2;
  float inv_scale_log2;
  int32_t num_kv_heads, n_rep, tpw, bs_log2;
  uint32_t num_blocks_u32;
  int32_t lane_offsets_32;  // 16 chunk rows of K and of V span < 2 GiB: 32-bit lane offsets
  // Key split: work items of 8 ints whose second half is (first key, end
  // key, unit, part | parts << 8 | max parts << 16); 4 ints: whole key
  // ranges, no split.
  int32_t item_ints;
  // The split's workspace: kPfMaxUnits int32 counters (parts done per
  // unit, zero at rest), then per unit max_parts blocks of kRowWaves * tpw
  // * n_rep records (D normalised fp32 values, the fp32 (max, sum) pair).
  // num_units / max_parts are the host-checked sizes it was allocated for;
  // an item outside them is skipped, never addressed.
  char* ws;
  int32_t num_units, max_parts;
};

template <int DTYPE, int D, typename BT>
__global__ __launch_bounds__((PfTraits<DTYPE, D>::kWaves * 64)) void paged_prefill_kernel(PrefillArgs a) {
  using Tr = PfTraits<DTYPE, D>;
  using raw_t = typename Elem<DTYPE>::raw;
  constexpr int L = Tr::kLoads;
  constexpr int RP = Tr::kRowPieces;
  constexpr int QP = Tr::kLanePieces;
  constexpr int S = Tr::kStages;
  constexpr int R = Tr::kRows;
  constexpr int kPfWaves = Tr::kWaves;
  constexpr int kPfStageTokens = Tr::kStageTokens;
  constexpr int U = Tr::kSetTiles;

  __shared__ __attribute__((aligned(16))) char s_lds[Tr::kLdsBytes];
  int32_t* s_ids = reinterpret_cast<int32_t*>(s_lds + Tr::kIdsOffset);
  const uint32_t lds0 = lds_address(s_lds);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int t = lane & 15;  // MFMA: key row (K operand) / query row (results)
  const int g = lane >> 4;  // MFMA: dim quarter (K operand) / key quad (results)
  const int rwave = Tr::kSets == 1 ? wave : wave % Tr::kRowWaves;  // rows
  const int set = Tr::kSets == 1 ? 0 : wave / Tr::kRowWaves;       // sub-tiles set * U .. of every stage

  const int4 w = reinterpret_cast<const int4*>(a.work)[blockIdx.x * (a.item_ints >> 2)];
  if (w.x < 0) return;  // an unused slot of a launch of fixed size
  const int seq = w.x, h = w.y, tok0 = w.z, ntok = w.w;
  // the key range of a split unit (its part number and count are read
  // again after the key loop, where they are used: registers are full)
  int kb0 = 0, kb1 = INT_MAX;
  if (a.item_ints == 8) {
    const int4 w2 = reinterpret_cast<const int4*>(a.work)[blockIdx.x * 2 + 1];
    kb0 = w2.x;
    kb1 = w2.y;
    // a part must address a record block of the workspace the host sized
    const int unit = w2.z, part = w2.w & 0xff, nparts = (w2.w >> 8) & 0xff;
    if (nparts < 1 || part >= nparts ||
        (nparts > 1 && (a.ws == nullptr || unit < 0 || unit >= a.num_units || nparts > a.max_parts)))
      return;
  }
  const int64_t row = a.seqs[4 * seq];
  const int cached = static_cast<int>(a.seqs[4 * seq + 1]);
  const int64_t qbase = a.seqs[4 * seq + 2] + tok0;  // chunk row of token tok0
  // keys of this work group: [kb0, key_end); the rows see keys below
  // cached + tok0 + ntok, and a part ends at a stage boundary below that
  const int key_end = min(cached + tok0 + ntok, kb1);
  const int bs_mask = (1 << a.bs_log2) - 1;

  // ---- rows of this wave: limits and Q (registers, straight from HBM)
  const int wtok0 = rwave * a.tpw;
  const int wtok_end = min(ntok, wtok0 + a.tpw);
  // the last key any row of the wave sees (-1: the wave has no rows)
  const int wave_limit = wtok0 < ntok ? cached + tok0 + wtok_end - 1 : -1;
  int limit[R];
  uint4 qr[R][QP];
#pragma unroll
  for (int rt = 0; rt < R; ++rt) {
    const int r = rt * 16 + t;
    const int rtok = wtok0 + r / a.n_rep;
    const bool ok = r < a.tpw * a.n_rep && rtok < ntok;
    limit[rt] = ok ? cached + tok0 + rtok : -1;  // -1: a padding row, never written
    const int tq = ok ? rtok : 0;
    const int head = h * a.n_rep + (ok ? r % a.n_rep : 0);
    const char* qrow = reinterpret_cast<const char*>(static_cast<const raw_t*>(a.q) +
                                                     (qbase + tq) * a.q_st + head * a.q_sh);
#pragma unroll
    for (int c = 0; c < QP; ++c) {
      qr[rt][c] = *reinterpret_cast<const uint4*>(qrow + (g * QP + c) * 16);
      // a padding row's Q is zero: finite scores, never written
      if (!ok) qr[rt][c] = uint4{0, 0, 0, 0};
    }
  }
  // Q must have landed before the tile copies are counted by vmcnt.
#pragma unroll
  for (int rt = 0; rt < R; ++rt)
#pragma unroll
    for (int c = 0; c < QP; ++c)
      asm volatile("" ::"v"(qr[rt][c].x), "v"(qr[rt][c].y), "v"(qr[rt][c].z), "v"(qr[rt][c].w));

  int slot_row[L], slot_piece[L];
#pragma unroll
  for (int c = 0; c < L; ++c) {
    const int slot = 64 * c + lane;
    slot_row[c] = slot / RP;
    slot_piece[c] = (slot % RP) ^ piece_swizzle<RP>(slot_row[c]);
  }

  float m_run[R], l_run[R];
  f32x4 o[R][D / 16];
#pragma unroll
  for (int rt = 0; rt < R; ++rt) {
    // 16-bit types: the row's reference (finite, see compute_stage)
    m_run[rt] = DTYPE == MV_DTYPE_F32 ? kNegInf : 0.f;
    l_run[rt] = 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) o[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const BT* btp = static_cast<const BT*>(a.block_table);
  const int win_tokens = kPfIdCap << a.bs_log2;  // a multiple of the stage size
  int win_blk0 = 0;

  // Byte offset of this lane's copy slot c within one 16-token tile of a
  // pool block, and within 16 chunk rows of row stride `st` (computed where
  // used: keeping all of them live spills registers at head_dim 128).
  auto pool_lane = [&](int c) { return static_cast<uint32_t>(slot_row[c] * Tr::kRowBytes + slot_piece[c] * 16); };
  auto chunk_lane = [&](int c, int64_t st) { return static_cast<uint32_t>(slot_row[c] * st + slot_piece[c] * 16); };
  const unsigned all_valid = (1u << L) - 1;

  // Copies wave's sub-tile of stage k (keys 64k + 16 wave ..) into buffer ST;
  // returns the slots that hold a key of the work group. Always 2L loads.
  // Two wave-uniform cases take one base address in SGPRs and a 32-bit
  // offset per lane: 16 prefix keys in one pool block (block size >= 16),
  // and 16 chunk keys all below key_end; the rest (a sub-tile that
  // straddles the prefix end or key_end, or smaller blocks) computes each
  // lane's address.
  auto issue_sub = [&](int kb, uint32_t dst) __attribute__((always_inline)) -> unsigned {
    // (Not for 16-bit types at head_dim 128: their registers are full, and
    // the extra live offsets spill.)
    constexpr bool kUniformPaths = D == 64 || DTYPE == MV_DTYPE_F32;
    if (kUniformPaths && kb + kTile <= cached && a.bs_log2 >= 4) {
      const int id = __builtin_amdgcn_readfirstlane(s_ids[min((kb >> a.bs_log2) - win_blk0, kPfIdCap - 1)]);
      const bool ok = static_cast<uint32_t>(id) < a.num_blocks_u32;
      const int64_t row0 = ok ? ((static_cast<int64_t>(id) * a.num_kv_heads + h) << a.bs_log2) + (kb & bs_mask) : 0;
      const char* bk = a.k_cache + row0 * Tr::kRowBytes;
      const char* bv = a.v_cache + row0 * Tr::kRowBytes;
#pragma unroll
      for (int c = 0; c < L; ++c) {
        copy_to_lds_16B_sv(bk, pool_lane(c), __builtin_amdgcn_readfirstlane(dst + c * 1024));
        copy_to_lds_16B_sv(bv, pool_lane(c), __builtin_amdgcn_readfirstlane(dst + Tr::kTileBytes + c * 1024));
      }
      return ok ? all_valid : 0u;
    }
    if (kUniformPaths && kb >= cached && kb + kTile <= key_end && a.lane_offsets_32) {
      const int64_t cr0 = qbase - tok0 + (kb - cached);  // chunk row of key kb
      const char* bk = a.k_new + cr0 * a.k_st + h * a.k_sh;
      const char* bv = a.v_new + cr0 * a.v_st + h * a.v_sh;
#pragma unroll
      for (int c = 0; c < L; ++c) {
        copy_to_lds_16B_sv(bk, chunk_lane(c, a.k_st), __builtin_amdgcn_readfirstlane(dst + c * 1024));
        copy_to_lds_16B_sv(bv, chunk_lane(c, a.v_st), __builtin_amdgcn_readfirstlane(dst + Tr::kTileBytes + c * 1024));
      }
      return all_valid;
    }
    unsigned valid = 0;
    const char* srck[L];
    const char* srcv[L];
#pragma unroll
    for (int c = 0; c < L; ++c) {
      const int j = kb + slot_row[c];
      bool ok = j < key_end;
      int64_t offk = slot_piece[c] * 16, offv = offk;
      const char* bk = a.k_cache;
      const char* bv = a.v_cache;
      if (j < cached) {
        const int id = s_ids[min((j >> a.bs_log2) - win_blk0, kPfIdCap - 1)];
        ok = ok && static_cast<uint32_t>(id) < a.num_blocks_u32;
        const int64_t rowoff = (((static_cast<int64_t>(id) * a.num_kv_heads + h) << a.bs_log2) +
                                (j & bs_mask)) * Tr::kRowBytes;
        offk += ok ? rowoff : 0;
        offv = offk;
      } else if (ok) {
        const int64_t cr = qbase - tok0 + (j - cached);  // chunk row of key j
        offk += cr * a.k_st + h * a.k_sh;
        offv += cr * a.v_st + h * a.v_sh;
        bk = a.k_new;
        bv = a.v_new;
      }
      srck[c] = bk + offk;
      srcv[c] = bv + offv;
      valid |= ok ? (1u << c) : 0u;
    }
#pragma unroll
    for (int c = 0; c < L; ++c) {
      copy_to_lds_16B(srck[c], __builtin_amdgcn_readfirstlane(dst + c * 1024));
      copy_to_lds_16B(srcv[c], __builtin_amdgcn_readfirstlane(dst + Tr::kTileBytes + c * 1024));
    }
    return valid;
  };

  // The wave's sub-tiles j * kPfWaves + wave of stage k; slot bits j * L + c.
  auto issue = [&](int k, auto st_c) __attribute__((always_inline)) -> unsigned {
    constexpr int ST = decltype(st_c)::value;
    unsigned v = 0;
#pragma unroll
    for (int j = 0; j < Tr::kWaveTiles; ++j) {
      const int su = j * kPfWaves + wave;
      v |= issue_sub(k * kPfStageTokens + su * kTile, lds0 + ST * Tr::kStageBytes + su * Tr::kSubBytes)
           << (j * L);
    }
    return v;
  };

  // V slots of keys that were not loaded read pool row 0 instead: zero
  // them (P is 0 there, but 0 * NaN would not be).
  auto zero_invalid_v = [&](int st, unsigned valid) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < Tr::kWaveTiles; ++j) {
      char* vdst = s_lds + st * Tr::kStageBytes + (j * kPfWaves + wave) * Tr::kSubBytes + Tr::kTileBytes;
#pragma unroll
      for (int c = 0; c < L; ++c)
        if (!((valid >> (j * L + c)) & 1u))
          *reinterpret_cast<uint4*>(vdst + c * 1024 + lane * 16) = make_uint4(0, 0, 0, 0);
    }
  };

  // The smallest causal limit among the wave's rows: a stage that ends at
  // or before it is seen whole by every row (no mask).
  const int wave_first_limit = cached + tok0 + wtok0;

  // One stage for this wave's rows, over the U sub-tiles of 16 keys of its
  // set (all kPfWaves sub-tiles with one set): S^T for every sub-tile some
  // row may see, one online-softmax update per row tile over the whole
  // stage, then O += P V per sub-tile.
  //
  // 16-bit types keep a per-row reference m (not necessarily the running
  // maximum; s and m in the exponent's units, s = scale * log2(e) * q.k)
  // with O and l relative to it. The QK^T MFMAs start from -m / (scale *
  // log2(e)) instead of 0, so one multiply turns their result into s - m.
  // A stage that no row's causal limit cuts ("whole") first tries
  // p = exp2(s - m) as it comes: no row maximum and no rescale of O (Q
  // itself is not scaled: rounding Q * scale * log2(e) to the data type
  // measured 0.077 max abs error against 0.016 on sharp bf16 scores, at
  // the same speed). It keeps that result when every
  // row's stage sum lies in [2^-12, 2^12] (so every p <= 2^12, within the
  // 16-bit types' range, and l stays well above underflow); otherwise, and
  // in the stages that cross the causal diagonal, the stage is computed
  // exactly: the row maximum d of s - m moves the reference by max(d, 0)
  // (by d while the row has seen no key), P and O are rescaled by it, and
  // P is rounded once, packed, for both the PV MFMA and the row sum.
  // (after_qk(): run once the stage's Q K^T MFMAs are issued, or at once
  // when the wave's rows see none of the stage's keys)
  auto compute_stage = [&](int k, int st, auto&& after_qk) __attribute__((always_inline)) {
    const int k_first = k * kPfStageTokens + set * U * kTile;  // the set's first key
    if (k_first > wave_limit) {  // causal: no row of the wave sees these keys
      after_qk();
      return;
    }
    // sub-tiles u < nu hold keys some row of the wave sees
    const int nu = min(U, (wave_limit - k_first) / kTile + 1);
    const bool whole = k_first + U * kTile - 1 <= wave_first_limit;  // then nu == U
    const char* stage = s_lds + st * Tr::kStageBytes + set * U * Tr::kSubBytes;
    const int ksw = piece_swizzle<RP>(t);
    f32x4 acc[U][R];
    // S^T - m (16-bit types; fp32: S^T) of the sub-tiles u < nu (u >= nu:
    // -m, never used unmasked). A whole stage has nu == U and branches on
    // no sub-tile.
    {
      f32x4 c0[R];
#pragma unroll
      for (int rt = 0; rt < R; ++rt) {
        const float c = DTYPE == MV_DTYPE_F32 ? 0.f : -m_run[rt] * a.inv_scale_log2;
        c0[rt] = f32x4{c, c, c, c};
      }
      auto qk_tile = [&](int u) __attribute__((always_inline)) {
        const char* k_tile = stage + u * Tr::kSubBytes;
#pragma unroll
        for (int c = 0; c < QP; ++c) {
          const uint4 kp = *reinterpret_cast<const uint4*>(k_tile + (t * RP + ((g * QP + c) ^ ksw)) * 16);
#pragma unroll
          for (int rt = 0; rt < R; ++rt) acc[u][rt] = mfma_qk<DTYPE>(kp, qr[rt][c], c == 0 ? c0[rt] : acc[u][rt]);
        }
      };
      if (whole) {
#pragma unroll
        for (int u = 0; u < U; ++u) qk_tile(u);
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (u < nu) {
            qk_tile(u);
          } else {
#pragma unroll
            for (int rt = 0; rt < R; ++rt) acc[u][rt] = c0[rt];
          }
        }
      }
    }
    after_qk();
    if constexpr (DTYPE == MV_DTYPE_F32) {
      float pr[U][R][4];
#pragma unroll
      for (int rt = 0; rt < R; ++rt) {
        float mc = kNegInf;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = k_first + u * kTile + 4 * g + e;
            const float sv = u < nu && key <= limit[rt] ? acc[u][rt][e] * a.scale_log2 : kNegInf;
            acc[u][rt][e] = sv;
            mc = fmaxf(mc, sv);
          }
        mc = fmaxf(mc, __shfl_xor(mc, 16));
        mc = fmaxf(mc, __shfl_xor(mc, 32));
        const float m_new = fmaxf(m_run[rt], mc);
        const float m_ref = m_new == kNegInf ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - m_ref);
        float lc = 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pr[u][rt][e] = __builtin_amdgcn_exp2f(acc[u][rt][e] - m_ref);
            lc += pr[u][rt][e];
          }
        lc += __shfl_xor(lc, 16);
        lc += __shfl_xor(lc, 32);
        l_run[rt] = l_run[rt] * alpha + lc;
        m_run[rt] = m_new;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float ar = __shfl(alpha, 4 * g + e);
#pragma unroll
          for (int c = 0; c < D / 16; ++c) o[rt][c][e] *= ar;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u < nu) mfma_pv_rows<DTYPE, D, R>(pr[u], stage + u * Tr::kSubBytes + Tr::kTileBytes, g, t, o);
    } else {
      // O += P V, sub-tile by sub-tile (past nu, P is 0 and every V slot
      // holds a pool row or zeros). At head_dim 64 the next sub-tile's V
      // operands are read while this one's MFMAs run (two operand sets in
      // flight: 41.9 against 42.5 us); at 128 a second set would not fit
      // the registers.
      auto pv = [&](s16x4 (&pk)[U][R], bool all) __attribute__((always_inline)) {
        if constexpr (D == 64 && MV_PREFILL_PV32) {
          // Two sub-tiles per 16x16x32 MFMA (half the MFMAs of 16x16x16).
#pragma unroll
          for (int u = 0; u < U; u += 2) {
            if (all || u < nu) {
              s16x4 va[D / 16], vb[D / 16];
              read_v_operands<DTYPE, D>(stage + u * Tr::kSubBytes + Tr::kTileBytes, g, t, va);
              read_v_operands<DTYPE, D>(stage + (u + 1) * Tr::kSubBytes + Tr::kTileBytes, g, t, vb);
              mfma_pv2_operands<DTYPE, D, R>(pk[u], pk[u + 1], va, vb, o);
            }
          }
        } else if constexpr (D == 64) {
          s16x4 vb[2][D / 16];
          read_v_operands<DTYPE, D>(stage + Tr::kTileBytes, g, t, vb[0]);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            if (all || u < nu) {
              if (u + 1 < U && (all || u + 1 < nu))
                read_v_operands<DTYPE, D>(stage + (u + 1) * Tr::kSubBytes + Tr::kTileBytes, g, t,
                                          vb[(u + 1) & 1]);
              __builtin_amdgcn_sched_barrier(0);
              mfma_pv_operands<DTYPE, D, R>(pk[u], vb[u & 1], o);
            }
          }
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u)
            if (all || u < nu)
              mfma_pv_packed<DTYPE, D, R>(pk[u], stage + u * Tr::kSubBytes + Tr::kTileBytes, g, t, o);
        }
      };
      // s - m in the exponent's units (+ b) from an MFMA result
      auto sc = [&](float x, float b = 0.f) __attribute__((always_inline)) {
        return __builtin_fmaf(x, a.scale_log2, b);
      };
      s16x4 pk[U][R];
      if (whole) {
        // p = exp2(s - m) as it comes; kept if every row's sum is in range
        float lc[R];
        bool out_of_range = false;
#pragma unroll
        for (int rt = 0; rt < R; ++rt) {
          lc[rt] = 0.f;
#pragma unroll
          for (int u = 0; u < U; ++u)
            pk[u][rt] = pack_p<DTYPE>(__builtin_amdgcn_exp2f(sc(acc[u][rt][0])), __builtin_amdgcn_exp2f(sc(acc[u][rt][1])),
                                      __builtin_amdgcn_exp2f(sc(acc[u][rt][2])), __builtin_amdgcn_exp2f(sc(acc[u][rt][3])),
                                      lc[rt]);
          lc[rt] += __shfl_xor(lc[rt], 16);
          lc[rt] += __shfl_xor(lc[rt], 32);
          // (a NaN sum fails both comparisons: it takes the exact path)
          out_of_range |= !(lc[rt] <= kPfFastMax && l_run[rt] + lc[rt] >= kPfFastMin);
        }
        if (__builtin_amdgcn_ballot_w64(out_of_range) == 0) {
#pragma unroll
          for (int rt = 0; rt < R; ++rt) l_run[rt] += lc[rt];
          pv(pk, true);
          return;
        }
        // (acc still holds s - m: the exact path below starts from it)
      }
      // exact: masked (the causal limit per row, recomputed here rather
      // than kept in registers), row maximum, reference moved, O rescaled
#pragma unroll
      for (int rt = 0; rt < R; ++rt) {
        int r = rt * 16 + t;
        asm volatile("" : "+v"(r));  // opaque to hoisting: a live copy per row tile costs registers
        const int rtok = wtok0 + r / a.n_rep;
        const int lim = r < a.tpw * a.n_rep && rtok < ntok ? cached + tok0 + rtok : -1;
        float mc = kNegInf;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = k_first + u * kTile + 4 * g + e;
            acc[u][rt][e] = u < nu && key <= lim ? acc[u][rt][e] : kNegInf;
            mc = fmaxf(mc, acc[u][rt][e]);
          }
        mc = fmaxf(mc, __shfl_xor(mc, 16));
        mc = sc(fmaxf(mc, __shfl_xor(mc, 32)));
        const bool seen = l_run[rt] > 0.f;
        const float shift = mc == kNegInf ? 0.f : seen ? fmaxf(mc, 0.f) : mc;
        const float alpha = seen ? __builtin_amdgcn_exp2f(-shift) : 0.f;  // O, l are 0 when unseen
        float lc = 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u)
          pk[u][rt] = pack_p<DTYPE>(__builtin_amdgcn_exp2f(sc(acc[u][rt][0], -shift)),
                                    __builtin_amdgcn_exp2f(sc(acc[u][rt][1], -shift)),
                                    __builtin_amdgcn_exp2f(sc(acc[u][rt][2], -shift)),
                                    __builtin_amdgcn_exp2f(sc(acc[u][rt][3], -shift)), lc);
        lc += __shfl_xor(lc, 16);
        lc += __shfl_xor(lc, 32);
        l_run[rt] = l_run[rt] * alpha + lc;
        m_run[rt] += shift;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float ar = __shfl(alpha, 4 * g + e);
#pragma unroll
          for (int c = 0; c < D / 16; ++c) o[rt][c][e] *= ar;
        }
      }
      pv(pk, false);
    }
  };

  // ---- windows of kPfIdCap prefix blocks (one window below 2048 blocks)
  // (first: the first key of the window's stages, a stage boundary)
  for (int first = kb0; first < key_end;) {
    const int win0 = first / win_tokens * win_tokens;
    win_blk0 = win0 >> a.bs_log2;
    if (win0 < cached) {
      const int pref_end = min(cached, win0 + win_tokens);
      const int nb = ((pref_end - 1) >> a.bs_log2) - win_blk0 + 1;
      for (int i = threadIdx.x; i < nb; i += kPfWaves * 64)
        s_ids[i] = static_cast<int32_t>(btp[row * a.bt_stride + win_blk0 + i]);
    }
    __syncthreads();  // block ids of the window visible; previous window's stages released
    const int k0 = first / kPfStageTokens;
    const int n = (min(key_end, win0 + win_tokens) - first + kPfStageTokens - 1) / kPfStageTokens;
    unsigned valid[S];
    valid[0] = issue(k0, IntC<0>{});
    if constexpr (S > 2) {
      if (1 < n) valid[1] = issue(k0 + 1, IntC<1>{});
    }
    // Stage i: wait for this wave's copies of it, clear its invalid V slots,
    // one barrier (every wave's part landed; stage i-1 consumed by all),
    // then refill stage i-1's buffer with stage i+S-1 and compute stage i.
    // With two sets, set 1 issues its copies after its Q K^T: the waves'
    // copy instructions then reach the CU's memory pipe in two rounds
    // instead of one, and set 1 starts its MFMAs at once (31.0 against
    // 31.7 us on a 4 x (1536 + 512) bf16 step; set 1 copying before P V
    // instead: 32.6 us).
    auto step = [&](int i, auto st_c) __attribute__((always_inline)) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int NX = (ST + S - 1) % S;
      wait_vmcnt_groups<2 * L * Tr::kWaveTiles, S - 2>(min(S - 2, n - 1 - i));
      asm volatile("" ::: "memory");
      // (only where a slot of this wave holds no key: a stage that straddles
      // the keys' end or the prefix end; 0.7 us of a 4 x (1536 + 512) bf16
      // step when it ran at every stage)
      if (__builtin_amdgcn_ballot_w64(valid[ST] != (1u << (L * Tr::kWaveTiles)) - 1u) != 0)
        zero_invalid_v(ST, valid[ST]);
      __syncthreads();
      const bool more = i + S - 1 < n;
      const bool late = Tr::kSets > 1 && set == 1;
      if (more && !late) valid[NX] = issue(k0 + i + S - 1, IntC<NX>{});
      asm volatile("" ::: "memory");
      compute_stage(k0 + i, ST, [&] {
        if (more && late) valid[NX] = issue(k0 + i + S - 1, IntC<NX>{});
        asm volatile("" ::: "memory");
      });
    };
    for (int i = 0; i < n; i += S) {
      step(i, IntC<0>{});
      if (i + 1 >= n) break;
      step(i + 1, IntC<1>{});
      if constexpr (S > 2) {
        if (i + 2 >= n) break;
        step(i + 2, IntC<2>{});
      }
    }
    __syncthreads();  // every wave is done with this window's stages and ids
    first = win0 + win_tokens;
  }

  if constexpr (DTYPE != MV_DTYPE_F32) {
    // a row that saw no key has no reference: the merges give it no weight
#pragma unroll
    for (int rt = 0; rt < R; ++rt)
      if (!(l_run[rt] > 0.f)) m_run[rt] = kNegInf;
  }

  // Lane coordinates recomputed for the epilogue rather than kept live
  // through the key loop (registers are full there).
  const int lane_e = __lane_id();
  const int te = lane_e & 15, ge = lane_e >> 4;

  // ---- merge the sets' softmax states (same rows): set s > 0 leaves m, l
  // and O in LDS (the stage buffers, free after the last barrier), set 0
  // folds them in and stores
  if constexpr (Tr::kSets > 1) {
    static_assert(Tr::kSets == 2, "two sets");
    float* xm = reinterpret_cast<float*>(s_lds) + rwave * Tr::kMergeFloats;  // m[R*16], l[R*16], O
    float* xo = xm + R * 32 + lane_e;
    if (set == 1) {
#pragma unroll
      for (int rt = 0; rt < R; ++rt) {
        if (ge == 0) {
          xm[rt * 16 + te] = m_run[rt];
          xm[R * 16 + rt * 16 + te] = l_run[rt];
        }
#pragma unroll
        for (int c = 0; c < D / 16; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) xo[((rt * (D / 16) + c) * 4 + e) * 64] = o[rt][c][e];
      }
    }
    __syncthreads();
    if (set == 0) {
#pragma unroll
    for (int rt = 0; rt < R; ++rt) {
      const float m1 = xm[rt * 16 + te];
      const float l1 = xm[R * 16 + rt * 16 + te];
      const float m = fmaxf(m_run[rt], m1);
      const float m_ref = m == kNegInf ? 0.f : m;
      const float a0 = __builtin_amdgcn_exp2f(m_run[rt] - m_ref);
      const float a1 = __builtin_amdgcn_exp2f(m1 - m_ref);
      l_run[rt] = l_run[rt] * a0 + l1 * a1;
      m_run[rt] = m;  // (max, sum) of both sets: a key-split part stores them
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a0r = __shfl(a0, 4 * ge + e);
        const float a1r = __shfl(a1, 4 * ge + e);
#pragma unroll
        for (int c = 0; c < D / 16; ++c)
          o[rt][c][e] = o[rt][c][e] * a0r + xo[((rt * (D / 16) + c) * 4 + e) * 64] * a1r;
      }
    }
    }
  }
  const bool rows_owner = Tr::kSets == 1 || set == 0;  // holds its rows' merged state

  // n_rep again, opaque to the compiler: its division constants are
  // recomputed here rather than held in a register through the key loop
  int n_rep_e = a.n_rep;
  asm volatile("" : "+s"(n_rep_e));
  // ---- normalise and store this wave's rows: to the output, or as this
  // part's partial rows (row index within the unit: token * n_rep + head)
  int unit = 0, part = 0, nparts = 1, max_parts = 1;
  if (a.item_ints == 8) {
    const int4 w2 = reinterpret_cast<const int4*>(a.work)[blockIdx.x * 2 + 1];
    unit = w2.z;
    part = w2.w & 0xff;
    nparts = (w2.w >> 8) & 0xff;
    max_parts = a.max_parts;  // the record stride the workspace was sized for
  }
  constexpr int kRec = D + 2;  // floats per record: the row, then (max, sum)
  const int rows_cap = Tr::kRowWaves * a.tpw * n_rep_e;
  float* recs = reinterpret_cast<float*>(a.ws + kPfCountersBytes) +
                static_cast<int64_t>(unit) * max_parts * rows_cap * kRec;
  int32_t* counter = reinterpret_cast<int32_t*>(a.ws) + unit;
  if (rows_owner) {
    const int64_t pbase = static_cast<int64_t>(part) * rows_cap + static_cast<int64_t>(rwave) * a.tpw * n_rep_e;
#pragma unroll
    for (int rt = 0; rt < R; ++rt) {
      const float inv = l_run[rt] > 0.f ? 1.f / l_run[rt] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rr = 4 * ge + e;  // row of o[rt][.][e]
        const float ir = __shfl(inv, rr);
        const int r = rt * 16 + rr;
        const int rtok = wtok0 + r / n_rep_e;
        if (r < a.tpw * n_rep_e && rtok < ntok) {
          if (nparts == 1) {
            raw_t* op = static_cast<raw_t*>(a.out) + (qbase + rtok) * a.o_st +
                        (h * n_rep_e + r % n_rep_e) * a.o_sh;
#pragma unroll
            for (int c = 0; c < D / 16; ++c) op[16 * c + te] = from_f32<DTYPE>(o[rt][c][e] * ir);
          } else {
            uint32_t* pp = reinterpret_cast<uint32_t*>(recs + (pbase + r) * kRec);
#pragma unroll
            for (int c = 0; c < D / 16; ++c) store_coherent_u32(pp + 16 * c + te, __float_as_uint(o[rt][c][e] * ir));
          }
        }
      }
      const int r = rt * 16 + te;  // the (max, sum) of row te, from the lanes ge == 0
      if (nparts > 1 && ge == 0 && r < a.tpw * n_rep_e && wtok0 + r / n_rep_e < ntok)
        store_coherent_u64(reinterpret_cast<uint64_t*>(recs + (pbase + r) * kRec + D), pack_f32x2(m_run[rt], l_run[rt]));
    }
  }
  if (nparts == 1) return;

  // ---- the part that completes the unit's count folds all parts: the
  // partial rows above are device-coherent stores; once every wave has seen
  // them acknowledged, the counter increment publishes them
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == nparts - 1;
  }
  __syncthreads();
  if (!s_last) return;
  constexpr int kRowThreads = D / 16;  // 16 dims (8 fp32 pairs) per thread
  const int nrows = ntok * n_rep_e;
  const int d0 = (threadIdx.x % kRowThreads) * 16;
  for (int gr = threadIdx.x / kRowThreads; gr < nrows; gr += kPfWaves * 64 / kRowThreads) {
    const float* rec0 = recs + static_cast<int64_t>(gr) * kRec;
    float m_all = kNegInf, l_all = 0.f;
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    // rounds of 4 parts, every load of a round in flight before the first use
    for (int p0 = 0; p0 < nparts; p0 += 4) {
      uint64_t ml[4], ov[4][8];
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const float* rec = rec0 + static_cast<int64_t>(min(p0 + pp, nparts - 1)) * rows_cap * kRec;
        ml[pp] = load_coherent_u64(reinterpret_cast<const uint64_t*>(rec + D));
        const uint64_t* src = reinterpret_cast<const uint64_t*>(rec + d0);
#pragma unroll
        for (int j = 0; j < 8; ++j) ov[pp][j] = load_coherent_u64(src + j);
      }
      float m_round = m_all;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp)
        if (p0 + pp < nparts) m_round = fmaxf(m_round, unpack_lo(ml[pp]));
      // every row sees key 0, which part 0 holds: m_round is finite
      const float rescale = m_all == kNegInf ? 0.f : __builtin_amdgcn_exp2f(m_all - m_round);
      l_all *= rescale;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] *= rescale;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const float mp = unpack_lo(ml[pp]);
        const float wgt = p0 + pp < nparts && mp != kNegInf
                              ? unpack_hi(ml[pp]) * __builtin_amdgcn_exp2f(mp - m_round) : 0.f;
        l_all += wgt;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          acc[2 * j] += wgt * unpack_lo(ov[pp][j]);
          acc[2 * j + 1] += wgt * unpack_hi(ov[pp][j]);
        }
      }
      m_all = m_round;
    }
    const float inv = 1.f / l_all;
    raw_t* op = static_cast<raw_t*>(a.out) + (qbase + gr / n_rep_e) * a.o_st +
                (h * n_rep_e + gr % n_rep_e) * a.o_sh + d0;
#pragma unroll
    for (int i = 0; i < 16; ++i) op[i] = from_f32<DTYPE>(acc[i] * inv);
  }
  if (threadIdx.x == 0)  // ready for the next call
    __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DTYPE, int D>
int launch_prefill(PrefillArgs a, int n_rep, int groups, bool bt_i64, hipStream_t s) {
  constexpr int kThreads = PfTraits<DTYPE, D>::kWaves * 64;
  a.tpw = pf_tokens_per_group<DTYPE, D>(n_rep) / PfTraits<DTYPE, D>::kRowWaves;
  if (bt_i64) paged_prefill_kernel<DTYPE, D, int64_t><<<groups, kThreads, 0, s>>>(a);
  else paged_prefill_kernel<DTYPE, D, int32_t><<<groups, kThreads, 0, s>>>(a);
  return check_launch("mv_paged_prefill");
}

template <template <int, int> class F>
int by_type(int head_dim, int dtype, int n_rep) {
  const bool d64 = head_dim == 64;
  switch (dtype) {
    case MV_DTYPE_F32: return d64 ? F<MV_DTYPE_F32, 64>::get(n_rep) : F<MV_DTYPE_F32, 128>::get(n_rep);
    case MV_DTYPE_F16: return d64 ? F<MV_DTYPE_F16, 64>::get(n_rep) : F<MV_DTYPE_F16, 128>::get(n_rep);
    default: return d64 ? F<MV_DTYPE_BF16, 64>::get(n_rep) : F<MV_DTYPE_BF16, 128>::get(n_rep);
  }
}
template <int DTYPE, int D>
struct TokensPerGroup {
  static int get(int n_rep) { return pf_tokens_per_group<DTYPE, D>(n_rep); }
};

template <int DTYPE>
int launch_prefill_d(const PrefillArgs& a, int d, int n_rep, int groups, bool bt_i64, hipStream_t s) {
  return d == 64 ? launch_prefill<DTYPE, 64>(a, n_rep, groups, bt_i64, s)
                 : launch_prefill<DTYPE, 128>(a, n_rep, groups, bt_i64, s);
}

}  // namespace
}  // namespace mv

namespace mv {
namespace {

// Device-side prefill plan for a launch of fixed size (graph capture, where
// the lengths cannot be read back): one work group validates each
// sequence's prefix entries, scans the chunk lengths into chunk rows, and
// writes the work list in sequence order, every slot past the last work
// group marked unused. status[0] = sequences with a bad row, length or
// prefix table entry; status[1] = work groups (or -1 when they exceed the
// capacity, or the chunk lengths the query rows: then every slot is unused).
constexpr int kPfPlanThreads = 256;
template <typename BT>
__global__ __launch_bounds__(kPfPlanThreads) void prefill_plan_kernel(
    const int64_t* rows, const int64_t* cached, const int64_t* qlen, int32_t num_seqs,
    int64_t total_rows, const BT* bt, int64_t bt_stride, int32_t bt_rows, int32_t max_blocks,
    int32_t bs_log2, int64_t num_blocks, int32_t tpg, int32_t num_kv_heads, int64_t* seqs,
    int32_t* work, int32_t work_cap, int32_t* status) {
  __shared__ int s_bad;
  __shared__ int64_t s_rows_total, s_groups;
  const int tid = threadIdx.x;
  if (tid == 0) {
    s_bad = 0;
    s_rows_total = 0;
    s_groups = 0;
  }
  __syncthreads();
  // 1. validate, sequence by sequence (prefill batches hold few sequences)
  for (int i = 0; i < num_seqs; ++i) {
    const int64_t r = rows[i], c = cached[i], q = qlen[i];
    const int64_t need = (c + (int64_t(1) << bs_log2) - 1) >> bs_log2;
    const bool shape_ok = r >= 0 && r < bt_rows && c >= 0 && q >= 0 && c <= INT_MAX / 2 &&
                          q <= INT_MAX / 2 && need <= max_blocks;
    int bad = 0;
    if (shape_ok) {
      for (int64_t j = tid; j < need; j += kPfPlanThreads) {
        const int64_t blk = static_cast<int64_t>(bt[r * bt_stride + j]);
        bad |= blk < 0 || blk >= num_blocks;
      }
    }
    bad = __syncthreads_or(bad);
    if (tid == 0) {
      if (!shape_ok || bad) ++s_bad;
      s_rows_total += q >= 0 ? q : 0;
      s_groups += q > 0 ? ((q + tpg - 1) / tpg) * num_kv_heads : 0;
    }
    __syncthreads();
  }
  const bool ok = s_bad == 0 && s_rows_total <= total_rows && s_groups <= work_cap;
  // 2. per-sequence rows and work groups (thread 0: a short sequential scan)
  if (tid == 0 && ok) {
    int64_t start = 0, slot = 0;
    for (int i = 0; i < num_seqs; ++i) {
      const int64_t q = qlen[i];
      seqs[4 * i] = rows[i];
      seqs[4 * i + 1] = cached[i];
      seqs[4 * i + 2] = start;
      seqs[4 * i + 3] = q;
      for (int64_t t0 = 0; t0 < q; t0 += tpg) {
        const int nt = static_cast<int>(q - t0 < tpg ? q - t0 : tpg);
        for (int h = 0; h < num_kv_heads; ++h, ++slot)
          reinterpret_cast<int4*>(work)[slot] = make_int4(i, h, static_cast<int>(t0), nt);
      }
      start += q;
    }
  }
  // 3. the unused slots (all of them for an unusable plan)
  const int64_t used = ok ? s_groups : 0;
  for (int64_t slot = used + tid; slot < work_cap; slot += kPfPlanThreads)
    reinterpret_cast<int4*>(work)[slot] = make_int4(-1, 0, 0, 0);
  if (tid == 0) {
    status[0] = s_bad;
    status[1] = ok ? static_cast<int32_t>(s_groups) : -1;
  }
}

}  // namespace
}  // namespace mv

extern "C" int mv_prefill_plan(const int64_t* seq_rows, const int64_t* cached_len,
                               const int64_t* query_len, int32_t num_seqs, int64_t total_query_rows,
                               const void* block_table, int32_t bt_is_i64, int64_t bt_stride,
                               int32_t bt_rows, int32_t max_blocks, int32_t block_size,
                               int64_t num_blocks, int32_t tokens_per_group, int32_t num_kv_heads,
                               int64_t* seqs, int32_t* work_items, int32_t work_capacity,
                               int32_t* status, void* stream) {
  using namespace mv;
  if (!status || !work_items || (num_seqs > 0 && (!seq_rows || !cached_len || !query_len || !seqs)))
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_prefill_plan: null pointer");
  if (num_seqs < 0 || work_capacity < 0 || tokens_per_group <= 0 || num_kv_heads <= 0 ||
      total_query_rows < 0 || bt_rows < 0 || max_blocks < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_prefill_plan: bad sizes");
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "mv_prefill_plan: block_size %d is not a power of 2", block_size);
  if (bt_rows > 0 && max_blocks > 0 && !block_table)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_prefill_plan: null block table");
  if (reinterpret_cast<uintptr_t>(work_items) % 16)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_prefill_plan: work_items not 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int bl = ilog2_exact(block_size);
  const int rows_ok = block_table ? bt_rows : 0;
  if (bt_is_i64)
    prefill_plan_kernel<int64_t><<<1, kPfPlanThreads, 0, s>>>(
        seq_rows, cached_len, query_len, num_seqs, total_query_rows,
        static_cast<const int64_t*>(block_table), bt_stride, rows_ok, max_blocks, bl, num_blocks,
        tokens_per_group, num_kv_heads, seqs, work_items, work_capacity, status);
  else
    prefill_plan_kernel<int32_t><<<1, kPfPlanThreads, 0, s>>>(
        seq_rows, cached_len, query_len, num_seqs, total_query_rows,
        static_cast<const int32_t*>(block_table), bt_stride, rows_ok, max_blocks, bl, num_blocks,
        tokens_per_group, num_kv_heads, seqs, work_items, work_capacity, status);
  return check_launch("mv_prefill_plan");
}

extern "C" int mv_prefill_tokens_per_group(int32_t num_q_heads, int32_t num_kv_heads,
                                           int32_t head_dim, int32_t dtype) {
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return 0;
  if ((head_dim != 64 && head_dim != 128) || mv::dtype_bytes(dtype) == 0) return 0;
  return mv::by_type<mv::TokensPerGroup>(head_dim, dtype, num_q_heads / num_kv_heads);
}

extern "C" size_t mv_paged_prefill_workspace_bytes(int32_t num_units, int32_t max_parts,
                                                   int32_t num_q_heads, int32_t num_kv_heads,
                                                   int32_t head_dim, int32_t dtype) {
  const int tpg = mv_prefill_tokens_per_group(num_q_heads, num_kv_heads, head_dim, dtype);
  if (tpg == 0 || num_units <= 0 || max_parts <= 1) return 0;
  const size_t rows = static_cast<size_t>(num_units) * max_parts * tpg * (num_q_heads / num_kv_heads);
  return mv::kPfCountersBytes + rows * (head_dim + 2) * 4;
}

namespace mv {
namespace {

// Key split of mv_paged_prefill_parts (null for mv_paged_prefill).
struct PrefillParts {
  int32_t num_units;
  int32_t max_parts;
  void* workspace;
  size_t workspace_bytes;
};

int paged_prefill(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                  const void* key, int64_t k_stride_tok, int64_t k_stride_head,
                  const void* value, int64_t v_stride_tok, int64_t v_stride_head,
                  const void* key_cache, const void* value_cache, const void* block_table,
                  int32_t bt_is_i64, int64_t bt_stride, const int64_t* seqs, int32_t num_seqs,
                  const int32_t* work_items, int32_t num_work_groups, void* out,
                  int64_t out_stride_tok, int64_t out_stride_head, float scale,
                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                  int32_t block_size, int64_t num_blocks, int32_t dtype,
                  const PrefillParts* parts, void* stream) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(MV_ERR_UNSUPPORTED, "mv_paged_prefill: unknown dtype %d", dtype);
  if (head_dim != 64 && head_dim != 128)
    return fail(MV_ERR_UNSUPPORTED, "mv_paged_prefill: head_dim %d not supported (64, 128)", head_dim);
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "mv_paged_prefill: block_size %d is not a power of 2", block_size);
  const int tpg = mv_prefill_tokens_per_group(num_q_heads, num_kv_heads, head_dim, dtype);
  if (tpg == 0)
    return fail(MV_ERR_UNSUPPORTED, "mv_paged_prefill: %d query heads over %d kv heads not supported",
                num_q_heads, num_kv_heads);
  if (num_seqs < 0 || num_work_groups < 0 || num_blocks <= 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_prefill: bad sizes");
  if (num_work_groups == 0) return MV_OK;
  if (!query || !key || !value || !key_cache || !value_cache || !seqs || !work_items || !out ||
      (!block_table && bt_stride != 0))
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_prefill: null pointer");
  if ((reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(key) |
       reinterpret_cast<uintptr_t>(value) | reinterpret_cast<uintptr_t>(key_cache) |
       reinterpret_cast<uintptr_t>(value_cache) | reinterpret_cast<uintptr_t>(work_items)) % 16 ||
      ((q_stride_tok | q_stride_head | k_stride_tok | k_stride_head | v_stride_tok |
        v_stride_head) * eb) % 16)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_paged_prefill: query/key/value rows and caches must be 16-byte aligned");
  PrefillArgs a;
  a.work = work_items;
  a.seqs = seqs;
  a.q = query;
  a.k_new = static_cast<const char*>(key);
  a.v_new = static_cast<const char*>(value);
  a.k_cache = static_cast<const char*>(key_cache);
  a.v_cache = static_cast<const char*>(value_cache);
  a.block_table = block_table;
  a.out = out;
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.k_st = k_stride_tok * eb;
  a.k_sh = k_stride_head * eb;
  a.v_st = v_stride_tok * eb;
  a.v_sh = v_stride_head * eb;
  a.o_st = out_stride_tok;
  a.o_sh = out_stride_head;
  a.bt_stride = bt_stride;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.inv_scale_log2 = 1.f / a.scale_log2;
  a.num_kv_heads = num_kv_heads;
  a.n_rep = num_q_heads / num_kv_heads;
  a.tpw = 0;  // set per instantiation at launch
  a.bs_log2 = ilog2_exact(block_size);
  a.num_blocks_u32 = static_cast<uint32_t>(std::min<int64_t>(num_blocks, int64_t(1) << 31));
  {
    const int64_t span = 16 * std::max(std::abs(a.k_st), std::abs(a.v_st)) + 16 * head_dim * eb;
    a.lane_offsets_32 = a.k_st >= 0 && a.v_st >= 0 && span < (int64_t(1) << 31);
  }
  a.item_ints = 4;
  a.ws = nullptr;
  a.num_units = 0;
  a.max_parts = 1;
  if (parts) {
    a.item_ints = 8;
    if (parts->num_units < 0 || parts->num_units > kPfMaxUnits || parts->max_parts < 1 ||
        parts->max_parts > kPfMaxParts)
      return fail(MV_ERR_INVALID_ARGUMENT,
                  "mv_paged_prefill_parts: %d units of %d parts (at most %d units, %d parts)",
                  parts->num_units, parts->max_parts, kPfMaxUnits, kPfMaxParts);
    if (parts->max_parts > 1) {
      const size_t need = mv_paged_prefill_workspace_bytes(parts->num_units, parts->max_parts,
                                                           num_q_heads, num_kv_heads, head_dim, dtype);
      if (!parts->workspace || parts->workspace_bytes < need)
        return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_prefill_parts: workspace %zu bytes, need %zu",
                    parts->workspace_bytes, need);
      if (reinterpret_cast<uintptr_t>(parts->workspace) % 256)
        return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_prefill_parts: workspace not 256-byte aligned");
      a.ws = static_cast<char*>(parts->workspace);
      a.num_units = parts->num_units;
      a.max_parts = parts->max_parts;
    }
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool i64 = bt_is_i64 != 0;
  const int n_rep = num_q_heads / num_kv_heads;
  switch (dtype) {
    case MV_DTYPE_F32: return launch_prefill_d<MV_DTYPE_F32>(a, head_dim, n_rep, num_work_groups, i64, s);
    case MV_DTYPE_F16: return launch_prefill_d<MV_DTYPE_F16>(a, head_dim, n_rep, num_work_groups, i64, s);
    default: return launch_prefill_d<MV_DTYPE_BF16>(a, head_dim, n_rep, num_work_groups, i64, s);
  }
}

}  // namespace
}  // namespace mv

extern "C" int mv_paged_prefill(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                                const void* key, int64_t k_stride_tok, int64_t k_stride_head,
                                const void* value, int64_t v_stride_tok, int64_t v_stride_head,
                                const void* key_cache, const void* value_cache,
                                const void* block_table, int32_t bt_is_i64, int64_t bt_stride,
                                const int64_t* seqs, int32_t num_seqs, const int32_t* work_items,
                                int32_t num_work_groups, void* out, int64_t out_stride_tok,
                                int64_t out_stride_head, float scale, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int64_t num_blocks, int32_t dtype, void* stream) {
  return mv::paged_prefill(query, q_stride_tok, q_stride_head, key, k_stride_tok, k_stride_head,
                           value, v_stride_tok, v_stride_head, key_cache, value_cache, block_table,
                           bt_is_i64, bt_stride, seqs, num_seqs, work_items, num_work_groups, out,
                           out_stride_tok, out_stride_head, scale, num_q_heads, num_kv_heads,
                           head_dim, block_size, num_blocks, dtype, nullptr, stream);
}

extern "C" int mv_paged_prefill_parts(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                                      const void* key, int64_t k_stride_tok, int64_t k_stride_head,
                                      const void* value, int64_t v_stride_tok, int64_t v_stride_head,
                                      const void* key_cache, const void* value_cache,
                                      const void* block_table, int32_t bt_is_i64, int64_t bt_stride,
                                      const int64_t* seqs, int32_t num_seqs,
                                      const int32_t* work_items, int32_t num_work_groups,
                                      int32_t num_units, int32_t max_parts, void* out, int64_t out_stride_tok, int64_t out_stride_head,
                                      float scale, int32_t num_q_heads, int32_t num_kv_heads,
                                      int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                      int32_t dtype, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  const mv::PrefillParts parts{num_units, max_parts, workspace, workspace_bytes};
  return mv::paged_prefill(query, q_stride_tok, q_stride_head, key, k_stride_tok, k_stride_head,
                           value, v_stride_tok, v_stride_head, key_cache, value_cache, block_table,
                           bt_is_i64, bt_stride, seqs, num_seqs, work_items, num_work_groups, out,
                           out_stride_tok, out_stride_head, scale, num_q_heads, num_kv_heads,
                           head_dim, block_size, num_blocks, dtype, &parts, stream);
}
