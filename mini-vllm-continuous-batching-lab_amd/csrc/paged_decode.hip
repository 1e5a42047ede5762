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
//   partition in chunks of kWaves * TPW 16-token tiles; wave w owns tiles
//   [w*TPW, (w+1)*TPW) of every chunk. A chunk goes HBM -> registers ->
//   LDS tile; the registers are refilled with the next chunk while the
//   staged one is computed.
//
// Per tile (16 tokens x D) and wave, with lane = 16*g + t (g = 0..3):
//   * Coalesced loads: load instruction c of lane l fetches the 16-byte
//     chunk 64c + l of the tile's row-major bytes, so each instruction reads
//     1 KiB of contiguous HBM (a whole pool block row set when BS >= 16).
//     K and V tiles land in per-wave LDS tiles whose rows are padded by
//     16 bytes.
//   * S^T = K Q^T on MFMA (16x16x32 for 16-bit types, 16x16x4 for fp32):
//     A = K tile (M = tokens), read from LDS as row t, dims
//     [g*D/4, (g+1)*D/4); B = Q^T (N = query heads of the group, rows >=
//     n_rep zero) from registers. Both operands use the same k-slot -> dim
//     mapping, so the contraction covers all D dims whatever the hardware's
//     k order.
//   * The accumulator holds S^T[token 4g+e][head t] in lane (g, t), slot e
//     -- the A-operand layout of the P V MFMA (M = heads, K = tokens), so
//     the probabilities never leave registers.
//   * V needs K = tokens in each lane: it is read from its LDS tile
//     column-wise (rows 0,4,8,12 of a column read start 16 banks apart, so
//     the four lane groups never collide).
//   Softmax is online across chunks (one rescale per chunk) and exact
//   within a chunk. The kWaves wave results are merged through LDS.
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
#ifndef MV_DECODE_WAVE_BYTES
#define MV_DECODE_WAVE_BYTES 4096  // K bytes per wave per chunk
#endif
#ifndef MV_DECODE_WAVES_PER_SIMD
#define MV_DECODE_WAVES_PER_SIMD 1  // register budget hint (1 = compiler's choice)
#endif
constexpr int kWaves = MV_DECODE_WAVES;
constexpr int kTile = 16;
constexpr int kMaxGroup = 16;   // MFMA N: query heads per kv head
constexpr int kMaxParts = 256;  // partitions per sequence (the plan enforces it)
constexpr int kMergeLoads = 8;  // partial loads in flight per output element
constexpr float kNegInf = -__builtin_huge_valf();

template <int DTYPE, int D>
struct Traits {
  static constexpr int kElemBytes = Elem<DTYPE>::bytes;
  static constexpr int kRowBytes = D * kElemBytes;  // one token row of one head
  static constexpr int kTileBytes = kTile * kRowBytes;
  static constexpr int kTilesPerWave =
      kTileBytes >= MV_DECODE_WAVE_BYTES ? 1 : MV_DECODE_WAVE_BYTES / kTileBytes;
  static constexpr int kChunk = kWaves * kTilesPerWave * kTile;  // tokens per iteration
  static constexpr int kLoads = kTileBytes / (64 * 16);          // 16-byte loads per lane per tile
  static constexpr int kRowChunks = kRowBytes / 16;
  static constexpr int kLdsRow = kRowBytes + 16;
  static constexpr int kLdsTile = kTile * kLdsRow;
  static constexpr int kLaneElems = D / 4;                         // MFMA: dims per lane per token
  static constexpr int kLaneChunks = kLaneElems * kElemBytes / 16;  // 16-byte pieces of those
  static constexpr int kWaveLds = 2 * kTilesPerWave * kLdsTile;     // K and V tiles
  static constexpr int kMergeBytes = kWaves * kMaxGroup * D * 4;          // wave merge
  static constexpr int kPartsBytes = 2 * kMaxGroup * kMaxParts * 4;       // partition merge
  static constexpr int kLdsBytes0 = kWaves * kWaveLds > kMergeBytes ? kWaves * kWaveLds : kMergeBytes;
  static constexpr int kLdsBytes = kLdsBytes0 > kPartsBytes ? kLdsBytes0 : kPartsBytes;
};

struct DecodeArgs {
  const void* q;
  int64_t q_stride_tok, q_stride_head;  // elements
  const char* k_cache;
  const char* v_cache;
  const void* block_table;
  int64_t bt_stride;  // elements
  const int32_t* kv_len;
  const int32_t* work;  // (seq, partition) pairs
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

// O tile update for one 16-token tile: o[c] += P(16 heads x 16 tokens) V(16 tokens x 16 dims).
template <int DTYPE, int D, int LDS_ROW>
__device__ __forceinline__ void mfma_pv(const float (&p)[4], const char* v_tile, int g, int t,
                                        f32x4 (&o)[D / 16]) {
  if constexpr (DTYPE == MV_DTYPE_F32) {
    const float* vt = reinterpret_cast<const float*>(v_tile);
    constexpr int rs = LDS_ROW / 4;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float vv = vt[(4 * g + e) * rs + 16 * c + t];
        o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[e], vv, o[c], 0, 0, 0);
      }
    }
  } else {
    const uint16_t* vt = reinterpret_cast<const uint16_t*>(v_tile);
    constexpr int rs = LDS_ROW / 2;
    s16x4 pa;
#pragma unroll
    for (int e = 0; e < 4; ++e) pa[e] = static_cast<short>(from_f32<DTYPE>(p[e]));
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      s16x4 vb;
#pragma unroll
      for (int e = 0; e < 4; ++e) vb[e] = static_cast<short>(vt[(4 * g + e) * rs + 16 * c + t]);
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

template <int DTYPE, int D, typename BT>
__global__ __launch_bounds__(kWaves * 64)
__attribute__((amdgpu_waves_per_eu(MV_DECODE_WAVES_PER_SIMD))) void paged_decode_kernel(DecodeArgs a) {
  using Tr = Traits<DTYPE, D>;
  using raw_t = typename Elem<DTYPE>::raw;
  constexpr int TPW = Tr::kTilesPerWave;
  constexpr int L = Tr::kLoads;
  constexpr int QC = Tr::kLaneChunks;

  __shared__ __attribute__((aligned(16))) char s_lds[Tr::kLdsBytes];
  __shared__ float s_max[kWaves][kMaxGroup];
  __shared__ float s_sum[kWaves][kMaxGroup];
  __shared__ int s_last;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = lane & 15;  // MFMA: token row (K operand) / head column (results)
  const int g = lane >> 4;  // MFMA: dim quarter (K operand) / token quad (results)

  const int item = blockIdx.x / a.num_kv_heads;
  const int h = blockIdx.x - item * a.num_kv_heads;
  const int b = a.work[2 * item];
  const int part = a.work[2 * item + 1];
  const int kv = a.kv_len[b];
  const int n_parts = (kv + a.part_tokens - 1) / a.part_tokens;
  const int tok_begin = part * a.part_tokens;
  const int tok_end = min(kv, tok_begin + a.part_tokens);
  const int n_chunks = (tok_end - tok_begin + Tr::kChunk - 1) / Tr::kChunk;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const BT* bt_row = static_cast<const BT*>(a.block_table) + b * a.bt_stride;

  char* k_lds = s_lds + wave * Tr::kWaveLds;
  char* v_lds = k_lds + TPW * Tr::kLdsTile;

  // Coalesced tile loads of chunk `ch`: piece 64c + lane of tile i.
  auto load_chunk = [&](int ch, uint4 (&kr)[TPW][L], uint4 (&vr)[TPW][L]) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile_tok = tok_begin + ch * Tr::kChunk + (wave * TPW + i) * kTile;
#pragma unroll
      for (int c = 0; c < L; ++c) {
        const int piece = 64 * c + lane;
        const int row = piece / Tr::kRowChunks;
        const int col = piece - row * Tr::kRowChunks;
        const int j = tile_tok + row;
        bool ok = j < tok_end;
        int64_t off = 0;
        if (ok) {
          const int64_t blk = static_cast<int64_t>(bt_row[j >> a.bs_log2]);
          ok = blk >= 0 && blk < a.num_blocks;  // the plan rejects such tables
          off = (((blk * a.num_kv_heads + h) << a.bs_log2) + (j & bs_mask)) * Tr::kRowBytes + col * 16;
        }
        kr[i][c] = ok ? *reinterpret_cast<const uint4*>(a.k_cache + off) : make_uint4(0, 0, 0, 0);
        vr[i][c] = ok ? *reinterpret_cast<const uint4*>(a.v_cache + off) : make_uint4(0, 0, 0, 0);
      }
    }
  };

  // ---- Q^T operand: head t of the group, dims of quarter g --------------
  uint4 qr[QC];
  {
    const bool ok = t < a.n_rep;
    const raw_t* qp = static_cast<const raw_t*>(a.q) + b * a.q_stride_tok +
                      (h * a.n_rep + (ok ? t : 0)) * a.q_stride_head + g * Tr::kLaneElems;
#pragma unroll
    for (int c = 0; c < QC; ++c)
      qr[c] = ok ? reinterpret_cast<const uint4*>(qp)[c] : make_uint4(0, 0, 0, 0);
  }

  float m_run = kNegInf;  // running max of head t (log2 domain)
  float l_run = 0.f;      // running sum of head t
  f32x4 o[D / 16];        // O[head 4g+e][dim 16c+t]
#pragma unroll
  for (int c = 0; c < D / 16; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Writes the chunk held in registers to the wave's LDS tiles.
  auto stage_chunk = [&](const uint4 (&kr)[TPW][L], const uint4 (&vr)[TPW][L]) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
#pragma unroll
      for (int c = 0; c < L; ++c) {
        const int piece = 64 * c + lane;
        const int row = piece / Tr::kRowChunks;
        const int col = piece - row * Tr::kRowChunks;
        const int lo = i * Tr::kLdsTile + row * Tr::kLdsRow + col * 16;
        *reinterpret_cast<uint4*>(k_lds + lo) = kr[i][c];
        *reinterpret_cast<uint4*>(v_lds + lo) = vr[i][c];
      }
    }
  };

  // Attention over the chunk staged in LDS (online softmax update).
  auto compute_chunk = [&](int ch) {
    // S^T = K Q^T
    float s[TPW][4];
    float mc = kNegInf;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const char* krow = k_lds + i * Tr::kLdsTile + t * Tr::kLdsRow + g * (Tr::kLaneElems * Tr::kElemBytes);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < QC; ++c) acc = mfma_qk<DTYPE>(reinterpret_cast<const uint4*>(krow)[c], qr[c], acc);
      const int tile_tok = tok_begin + ch * Tr::kChunk + (wave * TPW + i) * kTile;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s[i][e] = tile_tok + 4 * g + e < tok_end ? acc[e] * a.scale_log2 : kNegInf;
        mc = fmaxf(mc, s[i][e]);
      }
    }
    // head t's max over the chunk: lanes t, t+16, t+32, t+48
    mc = fmaxf(mc, __shfl_xor(mc, 16));
    mc = fmaxf(mc, __shfl_xor(mc, 32));
    const float m_new = fmaxf(m_run, mc);
    const float m_ref = m_new == kNegInf ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_ref);

    // P = exp2(S - m), rounded to the MFMA input type; the sum uses the
    // rounded values so O / l is an exact convex combination of V rows.
    float p[TPW][4];
    float lc = 0.f;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[i][e] = to_f32<DTYPE>(from_f32<DTYPE>(__builtin_amdgcn_exp2f(s[i][e] - m_ref)));
        lc += p[i][e];
      }
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
    // O += P V
#pragma unroll
    for (int i = 0; i < TPW; ++i) mfma_pv<DTYPE, D, Tr::kLdsRow>(p[i], v_lds + i * Tr::kLdsTile, g, t, o);
  };

  // ---- chunk loop: the next chunk's loads are in flight while the staged
  // chunk is computed (registers -> LDS tile -> registers refill) ---------
  {
    uint4 kr[TPW][L], vr[TPW][L];
    load_chunk(0, kr, vr);
    for (int ch = 0; ch < n_chunks; ++ch) {
      stage_chunk(kr, vr);
      wave_lds_order();
      if (ch + 1 < n_chunks) load_chunk(ch + 1, kr, vr);
      compute_chunk(ch);
      wave_lds_order();  // the next iteration overwrites the tiles
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
  // (max, sum) of every partial of the group's heads -> LDS in one round of
  // loads; per-head normalised weights; then each output element streams
  // its partials kMergeLoads at a time.
  float* s_m = reinterpret_cast<float*>(s_lds);  // [n_rep][n_parts]
  float* s_w = s_m + kMaxGroup * kMaxParts;      // [n_rep][n_parts]
  const int n_ml = a.n_rep * n_parts;
  for (int i = threadIdx.x; i < n_ml; i += kWaves * 64) {
    const int r = i / n_parts;
    const int64_t sl = slot_base + static_cast<int64_t>(r) * a.max_parts + (i - r * n_parts);
    s_m[i] = load_coherent(a.ws_ml + 2 * sl);
    s_w[i] = load_coherent(a.ws_ml + 2 * sl + 1);
  }
  __syncthreads();
  if (threadIdx.x < a.n_rep) {
    float* m_r = s_m + threadIdx.x * n_parts;
    float* w_r = s_w + threadIdx.x * n_parts;
    float mx = kNegInf;
    for (int p = 0; p < n_parts; ++p) mx = fmaxf(mx, m_r[p]);
    float sum = 0.f;
    for (int p = 0; p < n_parts; ++p) {
      w_r[p] *= __builtin_amdgcn_exp2f(m_r[p] - mx);
      sum += w_r[p];
    }
    const float inv = 1.f / sum;
    for (int p = 0; p < n_parts; ++p) w_r[p] *= inv;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < n_out; idx += kWaves * 64) {
    const int r = idx / D;
    const int d = idx - r * D;
    const int64_t s0 = slot_base + static_cast<int64_t>(r) * a.max_parts;
    const float* w_r = s_w + r * n_parts;
    float acc = 0.f;
    for (int p0 = 0; p0 < n_parts; p0 += kMergeLoads) {
      float ov[kMergeLoads];
#pragma unroll
      for (int u = 0; u < kMergeLoads; ++u)
        ov[u] = p0 + u < n_parts ? load_coherent(a.ws_o + (s0 + p0 + u) * D + d) : 0.f;
#pragma unroll
      for (int u = 0; u < kMergeLoads; ++u)
        if (p0 + u < n_parts) acc += w_r[p0 + u] * ov[u];
    }
    raw_t* op = static_cast<raw_t*>(a.out) + b * a.out_stride_tok + (h * a.n_rep + r) * a.out_stride_head;
    op[d] = from_f32<DTYPE>(acc);
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
  const int per_part = static_cast<int>(std::max<int64_t>(
      std::max<int64_t>(1, groups / std::max(1, a.target_groups)),
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
        a.work[2 * idx] = b;
        a.work[2 * idx + 1] = p;
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

template <int DTYPE, int D>
int chunk_of() { return Traits<DTYPE, D>::kChunk; }

int chunk_tokens(int head_dim, int dtype) {
  const bool d64 = head_dim == 64;
  switch (dtype) {
    case MV_DTYPE_F32: return d64 ? chunk_of<MV_DTYPE_F32, 64>() : chunk_of<MV_DTYPE_F32, 128>();
    case MV_DTYPE_F16: return d64 ? chunk_of<MV_DTYPE_F16, 64>() : chunk_of<MV_DTYPE_F16, 128>();
    default: return d64 ? chunk_of<MV_DTYPE_BF16, 64>() : chunk_of<MV_DTYPE_BF16, 128>();
  }
}

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
