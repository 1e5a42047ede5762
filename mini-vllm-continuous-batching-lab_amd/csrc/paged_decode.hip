// Paged-attention decode for gfx950 (MI355X), wave64 + MFMA.
//
// Math (AttentionBackendRef.decode_attention,
// mini_vllm/attention/paged_attention_ref.py:102-161):
//   out[b, hq] = softmax(scale * q[b, hq] . K_b[hk]^T) V_b[hk],
//   hk = hq / n_rep, n_rep = Hq / Hkv (repeat_interleave grouping),
//   token j of sequence b at block_table[b, j / BS], offset j % BS.
//
// Work decomposition
//   The context of every sequence is cut into partitions of kPartition
//   tokens. One work group of kWaves wavefronts handles one
//   (sequence, kv head, partition) and serves all n_rep query heads of the
//   GQA group, so every K/V byte is read from HBM exactly once.
//   Each wave owns kTilesPerWave consecutive 16-token tiles.
//
// Per tile (16 tokens x D) and wave, with lane = 16*g + t (g = 0..3):
//   * lane loads K[token t][g*D/4 .. (g+1)*D/4) straight from HBM into
//     registers (16-byte loads); the same for V.
//   * S^T = K Q^T on MFMA (16x16x32 for 16-bit types, 16x16x4 for fp32):
//     A = K tile (M = tokens), B = Q^T (N = query heads of the group,
//     rows >= n_rep are zero). The k-slot -> head_dim mapping is the same
//     for both operands, so the contraction is over all D dims whatever
//     the hardware's k order.
//   * The accumulator holds S^T[token 4g+e][head t] in lane (g, t), slot e
//     -- exactly the A-operand layout of the P V MFMA (M = heads,
//     K = tokens), so the probabilities never leave registers.
//   * V needs K = tokens in each lane, i.e. a transpose: the V tile goes
//     through a per-wave LDS tile (rows padded so the 4 lane groups hit
//     disjoint banks) and is read back column-wise.
//   Softmax is two-phase per wave (max over all of the wave's logits, then
//   exp2), so the accumulator is never rescaled inside a partition; the
//   kWaves partial results are merged through LDS at the end.
//   Sequences with one partition write the output directly; longer ones
//   write (normalised partial, max, sum) in fp32 and a second kernel merges
//   the partitions with a log-sum-exp reduce.
#include <algorithm>
#include <climits>

#include "mv_common.h"

namespace mv {
namespace {

constexpr int kWaves = 4;
constexpr int kTilesPerWave = 4;
constexpr int kTile = 16;
constexpr int kPartition = kWaves * kTilesPerWave * kTile;  // 256 tokens
constexpr int kMaxGroup = 16;                                 // MFMA N: q heads per kv head
constexpr float kNegInf = -__builtin_huge_valf();

struct DecodeArgs {
  const void* q;
  int64_t q_stride_tok, q_stride_head;  // elements
  const void* k_cache;
  const void* v_cache;
  const void* block_table;
  int64_t bt_stride;  // elements
  const int32_t* kv_len;
  const int32_t* work;  // (seq, partition) pairs
  void* out;
  int64_t out_stride_tok, out_stride_head;  // elements
  float* ws_o;                              // [num_seqs, Hq, max_parts, D]
  float2* ws_ml;                            // [num_seqs, Hq, max_parts]: (max, sum)
  float scale_log2;                         // scale * log2(e)
  int32_t num_q_heads, num_kv_heads, n_rep, bs_log2, max_parts;
  int64_t num_blocks;
};

template <typename BT>
__device__ __forceinline__ int64_t load_block_id(const BT* row, int idx) {
  return static_cast<int64_t>(row[idx]);
}

// --------------------------------------------------------------- MFMA ----

// S^T tile update: acc += K(16 tokens x 32 dims) * Q^T(32 dims x 16 heads)
// for the 16-bit types; one call per 16-byte chunk of the lane's dims.
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
  // 4 dims per 16-byte chunk, one 16x16x4 fp32 MFMA per dim slot.
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(k.x), __uint_as_float(q.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(k.y), __uint_as_float(q.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(k.z), __uint_as_float(q.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(k.w), __uint_as_float(q.w), acc, 0, 0, 0);
  return acc;
}

// ------------------------------------------------------- kernel traits ---

template <int DTYPE, int D>
struct Traits {
  static constexpr int kElemBytes = Elem<DTYPE>::bytes;
  static constexpr int kLaneElems = D / 4;                        // dims per lane per token
  static constexpr int kLaneChunks = kLaneElems * kElemBytes / 16;  // 16-byte loads per lane
  // LDS row of the V tile: D elements + pad. Rows 0,4,8,12 start 32 bytes
  // (16-bit) / 64 bytes (fp32) apart modulo the bank width, so the four
  // lane groups of a column read never share a bank.
  static constexpr int kPadBytes = kElemBytes == 2 ? 8 : 16;
  static constexpr int kRowBytes = D * kElemBytes + kPadBytes;
  static constexpr int kVTileBytes = kTile * kRowBytes;
  static constexpr int kMergeBytes = kWaves * kMaxGroup * D * 4;
  static constexpr int kUnionBytes =
      (kWaves * kVTileBytes > kMergeBytes ? kWaves * kVTileBytes : kMergeBytes);
};

// ---------------------------------------------------- partition kernel ---

template <int DTYPE, int D, typename BT>
__global__ __launch_bounds__(kWaves * 64) void paged_decode_partition_kernel(DecodeArgs a) {
  using Tr = Traits<DTYPE, D>;
  using raw_t = typename Elem<DTYPE>::raw;
  constexpr int C = Tr::kLaneChunks;

  __shared__ __attribute__((aligned(16))) char s_union[Tr::kUnionBytes];
  __shared__ float s_max[kWaves][kMaxGroup];
  __shared__ float s_sum[kWaves][kMaxGroup];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = lane & 15;  // token row (loads) / head column (results)
  const int g = lane >> 4;  // dim quarter (loads) / token quad (results)

  const int item = blockIdx.x / a.num_kv_heads;
  const int h = blockIdx.x - item * a.num_kv_heads;
  const int b = a.work[2 * item];
  const int part = a.work[2 * item + 1];
  const int kv = a.kv_len[b];
  const int n_parts = (kv + kPartition - 1) / kPartition;
  const int tile0 = part * kPartition + wave * kTilesPerWave * kTile;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const BT* bt_row = static_cast<const BT*>(a.block_table) + b * a.bt_stride;
  const raw_t* kc = static_cast<const raw_t*>(a.k_cache);
  const raw_t* vc = static_cast<const raw_t*>(a.v_cache);

  // ---- issue every K and V load of the wave up front ------------------
  uint4 kr[kTilesPerWave][C];
  uint4 vr[kTilesPerWave][C];
#pragma unroll
  for (int i = 0; i < kTilesPerWave; ++i) {
    const int j = tile0 + i * kTile + t;
    bool ok = j < kv;
    int64_t base = 0;
    if (ok) {
      const int64_t blk = load_block_id(bt_row, j >> a.bs_log2);
      ok = blk >= 0 && blk < a.num_blocks;  // the plan rejects such tables
      base = (((blk * a.num_kv_heads + h) << a.bs_log2) + (j & bs_mask)) * D + g * Tr::kLaneElems;
    }
    const uint4* kp = reinterpret_cast<const uint4*>(kc + base);
    const uint4* vp = reinterpret_cast<const uint4*>(vc + base);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      kr[i][c] = ok ? kp[c] : make_uint4(0, 0, 0, 0);
      vr[i][c] = ok ? vp[c] : make_uint4(0, 0, 0, 0);
    }
  }

  // ---- Q^T operand: head t of the group, dims of quarter g --------------
  uint4 qr[C];
  {
    const bool ok = t < a.n_rep;
    const raw_t* qp = static_cast<const raw_t*>(a.q) + b * a.q_stride_tok +
                      (h * a.n_rep + (ok ? t : 0)) * a.q_stride_head + g * Tr::kLaneElems;
#pragma unroll
    for (int c = 0; c < C; ++c) qr[c] = ok ? reinterpret_cast<const uint4*>(qp)[c] : make_uint4(0, 0, 0, 0);
  }

  // ---- S^T = K Q^T ------------------------------------------------------
  float s[kTilesPerWave][4];
  float m = kNegInf;
#pragma unroll
  for (int i = 0; i < kTilesPerWave; ++i) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < C; ++c) acc = mfma_qk<DTYPE>(kr[i][c], qr[c], acc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = tile0 + i * kTile + 4 * g + e;
      s[i][e] = j < kv ? acc[e] * a.scale_log2 : kNegInf;
      m = fmaxf(m, s[i][e]);
    }
  }
  // Row max over the wave: lanes t, t+16, t+32, t+48 hold head t.
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));
  const float m_ref = m == kNegInf ? 0.f : m;

  // ---- P = exp2(S - m), rounded to the MFMA input type -------------------
  // The row sum uses the rounded values, so the result is an exact convex
  // combination of the V rows up to the fp32 accumulation.
  float l = 0.f;
  float p[kTilesPerWave][4];
#pragma unroll
  for (int i = 0; i < kTilesPerWave; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pe = __builtin_amdgcn_exp2f(s[i][e] - m_ref);
      p[i][e] = to_f32<DTYPE>(from_f32<DTYPE>(pe));
      l += p[i][e];
    }
  }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);

  // ---- O = P V, V transposed through LDS ---------------------------------
  char* v_tile = s_union + wave * Tr::kVTileBytes;
  f32x4 o[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int i = 0; i < kTilesPerWave; ++i) {
    // Row t of the tile, bytes [g*D*eb/4, (g+1)*D*eb/4).
    char* wrow = v_tile + t * Tr::kRowBytes + g * (Tr::kLaneElems * Tr::kElemBytes);
    if constexpr (Tr::kElemBytes == 2) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        reinterpret_cast<uint2*>(wrow)[2 * c] = make_uint2(vr[i][c].x, vr[i][c].y);
        reinterpret_cast<uint2*>(wrow)[2 * c + 1] = make_uint2(vr[i][c].z, vr[i][c].w);
      }
    } else {
#pragma unroll
      for (int c = 0; c < C; ++c) reinterpret_cast<uint4*>(wrow)[c] = vr[i][c];
    }
    // LDS accesses of one wave complete in issue order; the barrier only
    // stops the compiler from moving the reads above the writes.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    if constexpr (DTYPE == MV_DTYPE_F32) {
      const float* vt = reinterpret_cast<const float*>(v_tile);
      constexpr int rs = Tr::kRowBytes / 4;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float vv = vt[(4 * g + e) * rs + 16 * c + t];
          o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[i][e], vv, o[c], 0, 0, 0);
        }
      }
    } else {
      const uint16_t* vt = reinterpret_cast<const uint16_t*>(v_tile);
      constexpr int rs = Tr::kRowBytes / 2;
      s16x4 pa;
#pragma unroll
      for (int e = 0; e < 4; ++e) pa[e] = static_cast<short>(from_f32<DTYPE>(p[i][e]));
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
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the waves ------------------------------------------------------
  __syncthreads();  // every wave is done with its V tile (s_union is reused)
  float* s_o = reinterpret_cast<float*>(s_union);  // [kWaves][kMaxGroup][D]
  if (g == 0) {
    s_max[wave][t] = m;
    s_sum[wave][t] = l;
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
    const int hq = h * a.n_rep + r;
    if (n_parts == 1) {
      raw_t* op = static_cast<raw_t*>(a.out) + b * a.out_stride_tok + hq * a.out_stride_head;
      op[d] = from_f32<DTYPE>(acc / sum);
    } else {
      const int64_t slot = (static_cast<int64_t>(b) * a.num_q_heads + hq) * a.max_parts + part;
      a.ws_o[slot * D + d] = acc / sum;
      if (d == 0) a.ws_ml[slot] = make_float2(mx, sum);
    }
  }
}

// ---------------------------------------------------- partition reduce ---

struct ReduceArgs {
  const float* ws_o;
  const float2* ws_ml;
  const int32_t* kv_len;
  void* out;
  int64_t out_stride_tok, out_stride_head;
  int32_t num_q_heads, max_parts;
};

// One wave per (sequence, query head): out = sum_p w_p o_p / sum_p w_p with
// w_p = sum_p * exp2(max_p - max). Single-partition sequences were written
// by the partition kernel.
template <int DTYPE, int D>
__global__ __launch_bounds__(64) void paged_decode_reduce_kernel(ReduceArgs a) {
  using raw_t = typename Elem<DTYPE>::raw;
  const int b = blockIdx.x / a.num_q_heads;
  const int hq = blockIdx.x - b * a.num_q_heads;
  const int kv = a.kv_len[b];
  const int n_parts = (kv + kPartition - 1) / kPartition;
  if (n_parts <= 1) return;
  const int64_t slot0 = (static_cast<int64_t>(b) * a.num_q_heads + hq) * a.max_parts;
  const float2* ml = a.ws_ml + slot0;
  float mx = kNegInf;
  for (int p = 0; p < n_parts; ++p) mx = fmaxf(mx, ml[p].x);
  constexpr int kPerLane = D / 64;
  float acc[kPerLane];
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) acc[k] = 0.f;
  float sum = 0.f;
  for (int p = 0; p < n_parts; ++p) {
    const float2 v = ml[p];
    const float w = v.y * __builtin_amdgcn_exp2f(v.x - mx);
    sum += w;
    const float* op = a.ws_o + (slot0 + p) * D;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) acc[k] += w * op[threadIdx.x + 64 * k];
  }
  raw_t* dst = static_cast<raw_t*>(a.out) + b * a.out_stride_tok + hq * a.out_stride_head;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) dst[threadIdx.x + 64 * k] = from_f32<DTYPE>(acc[k] / sum);
}

// ----------------------------------------------------------------- plan ---

struct PlanArgs {
  const void* kv_len;
  const void* block_table;
  int64_t bt_stride;
  int32_t num_seqs, max_blocks, bs_log2;
  int64_t num_blocks;
  int32_t* kv_out;
  int32_t* work;
  int64_t work_cap;
  int32_t* status;
};

constexpr int kPlanThreads = 1024;

template <typename KV, typename BT>
__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(PlanArgs a) {
  __shared__ int s_scan[kPlanThreads];
  __shared__ int s_cnt[4];  // bad kv_len, insufficient table, bad block id, max partitions
  __shared__ int s_min_kv;
  const int tid = threadIdx.x;
  if (tid < 4) s_cnt[tid] = 0;
  if (tid == 0) s_min_kv = INT_MAX;
  __syncthreads();

  const KV* kvp = static_cast<const KV*>(a.kv_len);
  const BT* btp = static_cast<const BT*>(a.block_table);
  const int64_t bs = int64_t(1) << a.bs_log2;
  int64_t running = 0;
  for (int base = 0; base < a.num_seqs; base += kPlanThreads) {
    const int b = base + tid;
    int np = 0;
    if (b < a.num_seqs) {
      const int64_t kv = static_cast<int64_t>(kvp[b]);
      int32_t kv32 = 0;
      atomicMin(&s_min_kv, static_cast<int>(std::max<int64_t>(std::min<int64_t>(kv, INT_MAX), INT_MIN)));
      if (kv < 1) {
        atomicAdd(&s_cnt[0], 1);
      } else if ((kv + bs - 1) / bs > a.max_blocks || kv > INT_MAX - kPartition) {
        atomicAdd(&s_cnt[1], 1);
      } else {
        kv32 = static_cast<int32_t>(kv);
        np = (kv32 + kPartition - 1) / kPartition;
        atomicMax(&s_cnt[3], np);
      }
      a.kv_out[b] = kv32;
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

  // Every table entry a valid sequence will read must be a pool block.
  const int64_t n = static_cast<int64_t>(a.num_seqs) * a.max_blocks;
  int bad = 0;
  for (int64_t i = tid; i < n; i += kPlanThreads) {
    const int64_t b = i / a.max_blocks;
    const int64_t j = i - b * a.max_blocks;
    const int64_t kv = static_cast<int64_t>(kvp[b]);
    if (kv < 1 || (kv + bs - 1) / bs > a.max_blocks) continue;
    if (j < (kv + bs - 1) / bs) {
      const int64_t blk = static_cast<int64_t>(btp[b * a.bt_stride + j]);
      bad += (blk < 0 || blk >= a.num_blocks);
    }
  }
  if (bad) atomicAdd(&s_cnt[2], bad);
  __syncthreads();
  if (tid == 0) {
    a.status[MV_PLAN_NUM_ITEMS] = static_cast<int32_t>(std::min<int64_t>(running, INT_MAX));
    a.status[MV_PLAN_BAD_KV_LEN] = s_cnt[0];
    a.status[MV_PLAN_INSUFFICIENT] = s_cnt[1];
    a.status[MV_PLAN_BAD_BLOCK] = s_cnt[2];
    a.status[MV_PLAN_MAX_PARTS] = s_cnt[3];
    a.status[MV_PLAN_MIN_KV_LEN] = a.num_seqs > 0 ? s_min_kv : 0;
    a.status[6] = 0;
    a.status[7] = 0;
  }
}

// ------------------------------------------------------------- dispatch ---

size_t ws_o_bytes(int64_t num_seqs, int64_t hq, int64_t d, int64_t parts) {
  return static_cast<size_t>(num_seqs * hq * parts * d * 4);
}

template <int DTYPE, int D, typename BT>
int launch_decode(const DecodeArgs& a, int num_items, int num_seqs, hipStream_t s) {
  if (num_items > 0) {
    const int64_t grid = static_cast<int64_t>(num_items) * a.num_kv_heads;
    if (grid > INT_MAX) return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: grid too large");
    paged_decode_partition_kernel<DTYPE, D, BT>
        <<<static_cast<unsigned>(grid), kWaves * 64, 0, s>>>(a);
  }
  if (a.max_parts > 1 && num_seqs > 0) {
    ReduceArgs r;
    r.ws_o = a.ws_o;
    r.ws_ml = a.ws_ml;
    r.kv_len = a.kv_len;
    r.out = a.out;
    r.out_stride_tok = a.out_stride_tok;
    r.out_stride_head = a.out_stride_head;
    r.num_q_heads = a.num_q_heads;
    r.max_parts = a.max_parts;
    paged_decode_reduce_kernel<DTYPE, D><<<num_seqs * a.num_q_heads, 64, 0, s>>>(r);
  }
  return check_launch("mv_paged_decode");
}

template <int DTYPE, int D>
int launch_decode_bt(const DecodeArgs& a, bool bt64, int num_items, int num_seqs, hipStream_t s) {
  return bt64 ? launch_decode<DTYPE, D, int64_t>(a, num_items, num_seqs, s)
              : launch_decode<DTYPE, D, int32_t>(a, num_items, num_seqs, s);
}

template <int DTYPE>
int launch_decode_d(const DecodeArgs& a, int d, bool bt64, int num_items, int num_seqs,
                    hipStream_t s) {
  return d == 64 ? launch_decode_bt<DTYPE, 64>(a, bt64, num_items, num_seqs, s)
                 : launch_decode_bt<DTYPE, 128>(a, bt64, num_items, num_seqs, s);
}

}  // namespace
}  // namespace mv

extern "C" int mv_decode_partition_tokens(void) { return mv::kPartition; }

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
                              int32_t* kv_len_i32, int32_t* work_items, int64_t work_capacity,
                              int32_t* status, void* stream) {
  using namespace mv;
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_plan: null status");
  if (num_seqs < 0 || max_blocks < 0 || work_capacity < 0 || num_blocks < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_plan: negative size");
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "mv_decode_plan: block_size %d is not a power of 2", block_size);
  if (num_seqs > 0 && (!kv_len || !kv_len_i32 || (max_blocks > 0 && !block_table)))
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
  a.num_blocks = num_blocks;
  a.kv_out = kv_len_i32;
  a.work = work_items;
  a.work_cap = work_capacity;
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
                               int32_t num_work_items, void* out, int64_t out_stride_tok,
                               int64_t out_stride_head, float scale, int32_t num_seqs,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t block_size, int64_t num_blocks, int32_t max_partitions,
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
  if (num_seqs == 0 || num_work_items == 0) return MV_OK;
  if (!query || !key_cache || !value_cache || !block_table || !kv_len_i32 || !work_items || !out)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: null pointer");
  // 16-byte loads of q rows and cache rows.
  const uintptr_t qa = reinterpret_cast<uintptr_t>(query);
  if ((qa | reinterpret_cast<uintptr_t>(key_cache) | reinterpret_cast<uintptr_t>(value_cache)) % 16 ||
      (q_stride_tok * eb) % 16 || (q_stride_head * eb) % 16)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: query/cache rows not 16-byte aligned");
  if (num_work_items > max_partitions * static_cast<int64_t>(num_seqs) && max_partitions > 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_paged_decode: work list larger than the plan allows");

  DecodeArgs a;
  a.q = query;
  a.q_stride_tok = q_stride_tok;
  a.q_stride_head = q_stride_head;
  a.k_cache = key_cache;
  a.v_cache = value_cache;
  a.block_table = block_table;
  a.bt_stride = bt_stride;
  a.kv_len = kv_len_i32;
  a.work = work_items;
  a.out = out;
  a.out_stride_tok = out_stride_tok;
  a.out_stride_head = out_stride_head;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.n_rep = n_rep;
  a.bs_log2 = ilog2_exact(block_size);
  a.max_parts = max_partitions;
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
    const size_t o = ws_o_bytes(num_seqs, num_q_heads, head_dim, max_partitions);
    a.ws_o = static_cast<float*>(workspace);
    a.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + ((o + 255) / 256) * 256);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bt64 = bt_is_i64 != 0;
  switch (dtype) {
    case MV_DTYPE_F32: return launch_decode_d<MV_DTYPE_F32>(a, head_dim, bt64, num_work_items, num_seqs, s);
    case MV_DTYPE_F16: return launch_decode_d<MV_DTYPE_F16>(a, head_dim, bt64, num_work_items, num_seqs, s);
    default: return launch_decode_d<MV_DTYPE_BF16>(a, head_dim, bt64, num_work_items, num_seqs, s);
  }
}
