// Fused rotary position embedding (RoPE) of one step's new tokens and the
// KV-cache write, for gfx950.
//
// One launch replaces three calls of QwenModelRunner.execute_model
// (mini_vllm/model_runner/qwen_runner.py:164-170):
//   q = rope(q, positions); k = rope(k, positions);
//   write_kv_cache(layer, k, v, slot_mapping)
// i.e. RotaryEmbedding.__call__ / _rotate_half (mini_vllm/model/rotary.py:
// 44-82) on the query and key heads, then the scatter of write_to_paged_cache
// (mini_vllm/cache/cache_write.py:25-74). The rotated key goes straight into
// its cache row; it is written to `key_out` as well only when the caller
// asks (prefill attention reads the new keys).
//
// Numerics are those of the reference's eager PyTorch ops in the tensors'
// dtype (mv_rope.h): the outputs are bit-identical to the reference's.
//
// Work split: a thread owns E = 16 / sizeof(elem) rotary pairs (d, d + D/2)
// of one (token, head): two 16-byte chunks of x, the matching chunks of the
// cos and sin rows of the token's position, two 16-byte stores (three with
// key_out). Query heads, key heads, then 16-byte value chunks (a bitwise
// copy into the cache) share one grid.
#include "mv_common.h"
#include "mv_rope.h"

namespace mv {
namespace {

struct RopeArgs {
  const char* q;
  char* q_out;
  const char* k;
  char* k_out;  // may be null
  const char* v;
  char* k_cache;
  char* v_cache;
  const int64_t* slots;
  const int64_t* positions;
  const char* cos;
  const char* sin;
  int64_t q_st, q_sh, qo_st, qo_sh, k_st, k_sh, ko_st, ko_sh, v_st, v_sh;  // bytes
  int64_t table_stride;  // bytes per cos / sin row
  int64_t max_positions;
  int64_t total_slots;
  int32_t num_tokens, num_q_heads, num_kv_heads, head_dim, block_size, bs_log2;
};

__device__ __forceinline__ int64_t cache_row(const RopeArgs& a, int64_t slot, int h) {
  const int64_t blk = slot >> a.bs_log2;
  const int64_t off = slot - (blk << a.bs_log2);
  return (blk * a.num_kv_heads + h) * a.block_size + off;  // rows of head_dim elements
}

template <int DTYPE>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(RopeArgs a) {
  using raw = typename Elem<DTYPE>::raw;
  constexpr int eb = sizeof(raw);
  constexpr int E = 16 / eb;  // rotary pairs per item
  const int half = a.head_dim / 2;
  const int per_head = half / E;
  const int heads = a.num_q_heads + a.num_kv_heads;
  const int n_rot = a.num_tokens * heads * per_head;
  const int v_chunks = a.head_dim / E;
  const int n_v = a.k_cache ? a.num_tokens * a.num_kv_heads * v_chunks : 0;
  const int total = n_rot + n_v;
  const int row_bytes = a.head_dim * eb;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    if (i < n_rot) {
      const int c = i % per_head;
      const int th = i / per_head;
      const int hh = th % heads;
      const int t = th / heads;
      int64_t pos = a.positions[t];
      pos = pos < 0 ? 0 : (pos >= a.max_positions ? a.max_positions - 1 : pos);  // checked on the host
      const bool is_q = hh < a.num_q_heads;
      const int h = is_q ? hh : hh - a.num_q_heads;
      const char* x = is_q ? a.q + t * a.q_st + h * a.q_sh : a.k + t * a.k_st + h * a.k_sh;
      const int o1 = c * E * eb, o2 = o1 + half * eb;  // byte offsets of the two halves
      const char* cr = a.cos + pos * a.table_stride;
      const char* sr = a.sin + pos * a.table_stride;
      const auto x1 = load16<DTYPE>(x + o1), x2 = load16<DTYPE>(x + o2);
      const auto c1 = load16<DTYPE>(cr + o1), c2 = load16<DTYPE>(cr + o2);
      const auto s1 = load16<DTYPE>(sr + o1), s2 = load16<DTYPE>(sr + o2);
      Chunk16<raw> y1, y2;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float u = to_f32<DTYPE>(x1.e[e]), w = to_f32<DTYPE>(x2.e[e]);
        y1.e[e] = rot_term<DTYPE, true>(u, to_f32<DTYPE>(c1.e[e]), w, to_f32<DTYPE>(s1.e[e]));
        y2.e[e] = rot_term<DTYPE, false>(w, to_f32<DTYPE>(c2.e[e]), u, to_f32<DTYPE>(s2.e[e]));
      }
      if (is_q) {
        char* out = a.q_out + t * a.qo_st + h * a.qo_sh;
        store16<DTYPE>(out + o1, y1);
        store16<DTYPE>(out + o2, y2);
      } else {
        if (a.k_out) {
          char* out = a.k_out + t * a.ko_st + h * a.ko_sh;
          store16<DTYPE>(out + o1, y1);
          store16<DTYPE>(out + o2, y2);
        }
        const int64_t slot = a.k_cache ? a.slots[t] : -1;
        if (slot >= 0 && slot < a.total_slots) {  // -1 skips; others are reported by the check
          char* dst = a.k_cache + cache_row(a, slot, h) * row_bytes;
          store16<DTYPE>(dst + o1, y1);
          store16<DTYPE>(dst + o2, y2);
        }
      }
    } else {
      const int r = i - n_rot;
      const int c = r % v_chunks;
      const int th = r / v_chunks;
      const int h = th % a.num_kv_heads;
      const int t = th / a.num_kv_heads;
      const uint4 val = *reinterpret_cast<const uint4*>(a.v + t * a.v_st + h * a.v_sh + c * 16);
      const int64_t slot = a.slots[t];
      if (slot >= 0 && slot < a.total_slots)
        *reinterpret_cast<uint4*>(a.v_cache + cache_row(a, slot, h) * row_bytes + c * 16) = val;
    }
  }
}

// status[0] = number of positions outside [0, max_positions).
__global__ __launch_bounds__(256) void positions_check_kernel(const int64_t* positions, int64_t n,
                                                              int64_t max_positions,
                                                              int32_t* status) {
  int bad = 0;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t p = positions[i];
    bad += p < 0 || p >= max_positions;
  }
  if (bad) atomicAdd(status, bad);
}

__global__ void zero_word(int32_t* status) {
  if (threadIdx.x == 0) status[0] = 0;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace mv

extern "C" int mv_rope_kv_cache_write(
    const void* query, int64_t q_stride_tok, int64_t q_stride_head, void* query_out,
    int64_t qo_stride_tok, int64_t qo_stride_head, const void* key, int64_t k_stride_tok,
    int64_t k_stride_head, void* key_out, int64_t ko_stride_tok, int64_t ko_stride_head,
    const void* value, int64_t v_stride_tok, int64_t v_stride_head, void* key_cache,
    void* value_cache, const int64_t* slot_mapping, const int64_t* positions,
    const void* cos_table, const void* sin_table, int64_t table_stride, int64_t max_positions,
    int64_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int64_t num_blocks, int32_t dtype, void* stream) {
  using namespace mv;
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(MV_ERR_UNSUPPORTED, "mv_rope_kv_cache_write: unknown dtype %d", dtype);
  const int E = 16 / eb;
  if (num_tokens < 0 || num_q_heads < 0 || num_kv_heads < 0 || head_dim <= 0 || max_positions <= 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_rope_kv_cache_write: bad sizes");
  if (head_dim % (2 * E))
    return fail(MV_ERR_UNSUPPORTED,
                "mv_rope_kv_cache_write: head_dim %d is not a multiple of %d for this dtype",
                head_dim, 2 * E);
  const bool write_cache = key_cache != nullptr;
  if (write_cache && (!value_cache || !slot_mapping || !value || num_blocks <= 0 ||
                      !is_pow2(block_size)))
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_rope_kv_cache_write: the cache write needs value, value_cache, slots, "
                "num_blocks > 0 and a power-of-two block_size (got %d)", block_size);
  if (num_tokens == 0 || num_q_heads + num_kv_heads == 0) return MV_OK;
  if (!positions || !cos_table || !sin_table || (num_q_heads > 0 && (!query || !query_out)) ||
      (num_kv_heads > 0 && !key))
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_rope_kv_cache_write: null pointer");
  // 16-byte chunks everywhere
  const void* ptrs[] = {query, query_out, key, key_out, value, key_cache, value_cache, cos_table, sin_table};
  for (const void* p : ptrs)
    if (p && !aligned16(p))
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_rope_kv_cache_write: pointers must be 16-byte aligned");
  const int64_t strides[] = {q_stride_tok, q_stride_head, qo_stride_tok, qo_stride_head, k_stride_tok,
                             k_stride_head, ko_stride_tok, ko_stride_head, v_stride_tok, v_stride_head,
                             table_stride};
  for (int64_t st : strides)
    if ((st * eb) % 16)
      return fail(MV_ERR_INVALID_ARGUMENT,
                  "mv_rope_kv_cache_write: strides must be multiples of 16 bytes");
  const int64_t heads = static_cast<int64_t>(num_q_heads) + num_kv_heads;
  const int64_t work = num_tokens * heads * (head_dim / 2 / E) +
                       (write_cache ? num_tokens * num_kv_heads * (head_dim / E) : 0);
  if (work >= INT_MAX - 65536LL * 256)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_rope_kv_cache_write: %lld tokens is too many",
                static_cast<long long>(num_tokens));

  RopeArgs a;
  a.q = static_cast<const char*>(query);
  a.q_out = static_cast<char*>(query_out);
  a.k = static_cast<const char*>(key);
  a.k_out = static_cast<char*>(key_out);
  a.v = static_cast<const char*>(value);
  a.k_cache = static_cast<char*>(key_cache);
  a.v_cache = static_cast<char*>(value_cache);
  a.slots = slot_mapping;
  a.positions = positions;
  a.cos = static_cast<const char*>(cos_table);
  a.sin = static_cast<const char*>(sin_table);
  a.q_st = q_stride_tok * eb;
  a.q_sh = q_stride_head * eb;
  a.qo_st = qo_stride_tok * eb;
  a.qo_sh = qo_stride_head * eb;
  a.k_st = k_stride_tok * eb;
  a.k_sh = k_stride_head * eb;
  a.ko_st = ko_stride_tok * eb;
  a.ko_sh = ko_stride_head * eb;
  a.v_st = v_stride_tok * eb;
  a.v_sh = v_stride_head * eb;
  a.table_stride = table_stride * eb;
  a.max_positions = max_positions;
  a.total_slots = write_cache ? num_blocks * block_size : 0;
  a.num_tokens = static_cast<int32_t>(num_tokens);
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.block_size = write_cache ? block_size : 1;
  a.bs_log2 = write_cache ? ilog2_exact(block_size) : 0;

  const int blocks = static_cast<int>(std::min<int64_t>((work + 255) / 256, 65536));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MV_DTYPE_F32: rope_kv_write_kernel<MV_DTYPE_F32><<<blocks, 256, 0, s>>>(a); break;
    case MV_DTYPE_F16: rope_kv_write_kernel<MV_DTYPE_F16><<<blocks, 256, 0, s>>>(a); break;
    default: rope_kv_write_kernel<MV_DTYPE_BF16><<<blocks, 256, 0, s>>>(a); break;
  }
  return check_launch("mv_rope_kv_cache_write");
}

extern "C" int mv_positions_check(const int64_t* positions, int64_t num_tokens,
                                  int64_t max_positions, int32_t* status, void* stream) {
  using namespace mv;
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "mv_positions_check: null status");
  if (num_tokens < 0) return fail(MV_ERR_INVALID_ARGUMENT, "mv_positions_check: negative size");
  if (num_tokens > 0 && !positions)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_positions_check: null positions");
  hipStream_t s = static_cast<hipStream_t>(stream);
  zero_word<<<1, 64, 0, s>>>(status);
  if (num_tokens > 0) {
    const int blocks = static_cast<int>(std::min<int64_t>((num_tokens + 255) / 256, 1024));
    positions_check_kernel<<<blocks, 256, 0, s>>>(positions, num_tokens, max_positions, status);
  }
  return check_launch("mv_positions_check");
}
