// KV-cache write (scatter by slot) and slot validation for gfx950.
//
// Follows write_to_paged_cache (mini_vllm/cache/cache_write.py:25-74) and
// replaces the Triton `_cache_write_kernel` (paged_attention_gpu.py:33-87).
//
// Layout of one token row: key[t, h, 0:D] sits at key + t*stride_tok +
// h*stride_head (elements) with the D elements contiguous; its destination
// is the contiguous D-element row cache[s / BS, h, s % BS, :].
//
// The write moves whole VEC-byte chunks (VEC = 16/8/4/2, the widest width
// that every address and stride allows), one chunk per thread, K chunks
// and V chunks in the same grid. It is a bitwise copy, so the result is
// bit-identical to the reference scatter for every dtype.
#include "mv_common.h"

namespace mv {
namespace {

template <int VEC> struct Chunk;
template <> struct Chunk<16> { using type = uint4; };
template <> struct Chunk<8> { using type = uint2; };
template <> struct Chunk<4> { using type = uint32_t; };
template <> struct Chunk<2> { using type = uint16_t; };

// Uses a loaded chunk in an empty asm (with a memory clobber, so loads
// issued before it stay before it): the compiler can then no longer sink
// the load below the slot check that guards the store.
__device__ __forceinline__ void keep_loaded(const uint4& v) {
  asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w) : "memory");
}
__device__ __forceinline__ void keep_loaded(const uint2& v) {
  asm volatile("" ::"v"(v.x), "v"(v.y) : "memory");
}
__device__ __forceinline__ void keep_loaded(uint32_t v) { asm volatile("" ::"v"(v) : "memory"); }
__device__ __forceinline__ void keep_loaded(uint16_t v) {
  asm volatile("" ::"v"(static_cast<uint32_t>(v)) : "memory");
}

struct WriteArgs {
  const char* key;
  const char* value;
  int64_t key_stride_tok, key_stride_head;      // bytes
  int64_t value_stride_tok, value_stride_head;  // bytes
  char* key_cache;
  char* value_cache;
  const int64_t* slots;
  int64_t num_tokens;
  int64_t total_slots;
  int32_t num_kv_heads;
  int32_t row_bytes;  // head_dim * element bytes
  int32_t block_size;
  int32_t bs_log2;    // log2(block_size) when it is a power of two, else -1
};

template <int VEC>
__global__ __launch_bounds__(256) void kv_cache_write_kernel(WriteArgs a) {
  using C = typename Chunk<VEC>::type;
  // 32-bit index math (the host guarantees 2 * rows * chunks < 2^31)
  const int chunks_per_row = a.row_bytes / VEC;
  const int rows = static_cast<int>(a.num_tokens) * a.num_kv_heads;
  const int per_tensor = rows * chunks_per_row;
  const int total = 2 * per_tensor;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const bool is_v = i >= per_tensor;
    const int r = is_v ? i - per_tensor : i;
    const int row = r / chunks_per_row;
    const int chunk = r - row * chunks_per_row;
    const int t = row / a.num_kv_heads;
    const int h = row - t * a.num_kv_heads;
    // The source chunk and the slot are loaded together: the source address
    // does not depend on the slot, so the copy costs one memory round trip.
    const char* src = is_v ? a.value + t * a.value_stride_tok + h * a.value_stride_head
                           : a.key + t * a.key_stride_tok + h * a.key_stride_head;
    const C v = reinterpret_cast<const C*>(src)[chunk];
    const int64_t slot = a.slots[t];
    keep_loaded(v);
    // -1 skips (prefix-cache hit); anything else outside the pool is
    // reported by the slot check and never written.
    if (slot < 0 || slot >= a.total_slots) continue;
    const int64_t blk = a.bs_log2 >= 0 ? slot >> a.bs_log2 : slot / a.block_size;
    const int64_t off = slot - blk * a.block_size;
    char* dst = (is_v ? a.value_cache : a.key_cache) +
                ((blk * a.num_kv_heads + h) * a.block_size + off) * a.row_bytes;
    reinterpret_cast<C*>(dst)[chunk] = v;
  }
}

// One work group compares a 256-slot tile `i` against tile `j >= i`.
// status[0] counts slots outside [-1, total_slots), status[1] counts pairs
// (x < y) of equal in-range slots. Counters start at zero (zero_status).
constexpr int kCheckTile = 256;

__global__ __launch_bounds__(kCheckTile) void slots_check_kernel(const int64_t* slots, int64_t n,
                                                                 int64_t total_slots,
                                                                 int32_t* status) {
  const int64_t ti = blockIdx.x, tj = blockIdx.y;
  if (tj < ti) return;
  __shared__ int64_t s_other[kCheckTile];
  __shared__ int s_dups, s_bad;
  if (threadIdx.x == 0) { s_dups = 0; s_bad = 0; }
  const int64_t y0 = tj * kCheckTile;
  const int64_t yi = y0 + threadIdx.x;
  s_other[threadIdx.x] = yi < n ? slots[yi] : -1;
  __syncthreads();
  const int64_t x = ti * kCheckTile + threadIdx.x;
  int dups = 0;
  if (x < n) {
    const int64_t s = slots[x];
    const bool in_range = s >= 0 && s < total_slots;
    if (ti == tj && !in_range && s != -1) atomicAdd(&s_bad, 1);
    if (in_range) {
      const int64_t lim = min<int64_t>(kCheckTile, n - y0);
      for (int k = 0; k < lim; ++k) {
        dups += (y0 + k > x) && (s_other[k] == s);
      }
    }
  }
  if (dups) atomicAdd(&s_dups, dups);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (s_bad) atomicAdd(&status[MV_SLOTS_OUT_OF_RANGE], s_bad);
    if (s_dups) atomicAdd(&status[MV_SLOTS_DUPLICATES], s_dups);
  }
}

// The fused decode + KV write (mv_paged_decode_write) is exact when every
// slot is -1 or the table position of its own sequence's last attended
// token kv_len - 1 (the block manager's layout). One work group counts the
// sequences for which that does not hold (including those with a kv_len or
// table entry that cannot address such a position) into status[0].
constexpr int kWriteCheckThreads = 256;
template <typename KV, typename BT>
__global__ __launch_bounds__(kWriteCheckThreads) void decode_write_check_kernel(
    const int64_t* slots, const BT* bt, int64_t bt_stride, const KV* kv_len, int32_t num_seqs,
    int32_t max_blocks, int32_t bs_log2, int32_t* status) {
  __shared__ int s_bad;
  if (threadIdx.x == 0) s_bad = 0;
  __syncthreads();
  int bad = 0;
  for (int b = threadIdx.x; b < num_seqs; b += kWriteCheckThreads) {
    const int64_t s = slots[b];
    if (s == -1) continue;
    const int64_t kv = static_cast<int64_t>(kv_len[b]);
    const int64_t e = (kv - 1) >> bs_log2;
    bool ok = kv >= 1 && e < max_blocks;
    if (ok) {
      const int64_t blk = static_cast<int64_t>(bt[b * bt_stride + e]);
      ok = blk >= 0 && s == (blk << bs_log2) + ((kv - 1) & ((int64_t(1) << bs_log2) - 1));
    }
    bad += !ok;
  }
  if (bad) atomicAdd(&s_bad, bad);
  __syncthreads();
  if (threadIdx.x == 0) status[0] = s_bad;
}

__global__ void zero_status(int32_t* status, int n) {
  if (threadIdx.x < n) status[threadIdx.x] = 0;
}

inline int pick_vec(int64_t row_bytes, std::initializer_list<int64_t> values) {
  for (int vec : {16, 8, 4, 2}) {
    bool ok = row_bytes % vec == 0;
    for (int64_t v : values) ok = ok && (v % vec == 0);
    if (ok) return vec;
  }
  return 0;
}

}  // namespace
}  // namespace mv

extern "C" int mv_kv_cache_write(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                                 const void* value, int64_t value_stride_tok,
                                 int64_t value_stride_head, void* key_cache, void* value_cache,
                                 const int64_t* slot_mapping, int64_t num_tokens,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                 int64_t num_blocks, int32_t dtype, void* stream) {
  using namespace mv;
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(MV_ERR_UNSUPPORTED, "mv_kv_cache_write: unknown dtype %d", dtype);
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks <= 0)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_kv_cache_write: bad sizes (num_tokens=%lld num_kv_heads=%d head_dim=%d "
                "block_size=%d num_blocks=%lld)",
                (long long)num_tokens, num_kv_heads, head_dim, block_size, (long long)num_blocks);
  if (num_tokens == 0) return MV_OK;
  if (!key || !value || !key_cache || !value_cache || !slot_mapping)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_cache_write: null pointer");

  WriteArgs a;
  a.key = static_cast<const char*>(key);
  a.value = static_cast<const char*>(value);
  a.key_stride_tok = key_stride_tok * eb;
  a.key_stride_head = key_stride_head * eb;
  a.value_stride_tok = value_stride_tok * eb;
  a.value_stride_head = value_stride_head * eb;
  a.key_cache = static_cast<char*>(key_cache);
  a.value_cache = static_cast<char*>(value_cache);
  a.slots = slot_mapping;
  a.num_tokens = num_tokens;
  a.total_slots = num_blocks * block_size;
  a.num_kv_heads = num_kv_heads;
  a.row_bytes = head_dim * eb;
  a.block_size = block_size;
  a.bs_log2 = is_pow2(block_size) ? ilog2_exact(block_size) : -1;

  const int vec = pick_vec(a.row_bytes,
                           {(int64_t)(uintptr_t)key, (int64_t)(uintptr_t)value,
                            (int64_t)(uintptr_t)key_cache, (int64_t)(uintptr_t)value_cache,
                            a.key_stride_tok, a.key_stride_head, a.value_stride_tok,
                            a.value_stride_head});
  if (vec == 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_cache_write: addresses not 2-byte aligned");

  const int64_t work = 2 * num_tokens * num_kv_heads * (a.row_bytes / vec);
  if (work >= INT_MAX)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_cache_write: %lld tokens x %d heads is too many",
                (long long)num_tokens, num_kv_heads);
  const int threads = 256;
  const int64_t blocks = std::min<int64_t>((work + threads - 1) / threads, 65536);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (vec) {
    case 16: kv_cache_write_kernel<16><<<blocks, threads, 0, s>>>(a); break;
    case 8: kv_cache_write_kernel<8><<<blocks, threads, 0, s>>>(a); break;
    case 4: kv_cache_write_kernel<4><<<blocks, threads, 0, s>>>(a); break;
    default: kv_cache_write_kernel<2><<<blocks, threads, 0, s>>>(a); break;
  }
  return check_launch("mv_kv_cache_write");
}

extern "C" int mv_kv_slots_check(const int64_t* slot_mapping, int64_t num_tokens,
                                 int64_t total_slots, int32_t* status, void* stream) {
  using namespace mv;
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_slots_check: null status");
  if (num_tokens < 0 || total_slots < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_slots_check: negative size");
  hipStream_t s = static_cast<hipStream_t>(stream);
  zero_status<<<1, 64, 0, s>>>(status, 2);
  if (num_tokens > 0) {
    if (!slot_mapping) return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_slots_check: null slots");
    const int64_t tiles = (num_tokens + kCheckTile - 1) / kCheckTile;
    if (tiles > 65535)
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_slots_check: %lld tokens is too many",
                  (long long)num_tokens);
    dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(tiles));
    slots_check_kernel<<<grid, kCheckTile, 0, s>>>(slot_mapping, num_tokens, total_slots, status);
  }
  return check_launch("mv_kv_slots_check");
}

extern "C" int mv_decode_write_check(const int64_t* slot_mapping, const void* block_table,
                                     int32_t bt_is_i64, int64_t bt_stride, const void* kv_len,
                                     int32_t kv_len_is_i64, int32_t num_seqs, int32_t max_blocks,
                                     int32_t block_size, int32_t* status, void* stream) {
  using namespace mv;
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_write_check: null status");
  if (num_seqs < 0 || max_blocks < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_write_check: negative size");
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "mv_decode_write_check: block_size %d is not a power of 2",
                block_size);
  if (num_seqs > 0 && (!slot_mapping || !kv_len || (max_blocks > 0 && !block_table)))
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_write_check: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int bl = ilog2_exact(block_size);
  const int mb = block_table ? max_blocks : 0;
  if (kv_len_is_i64) {
    if (bt_is_i64)
      decode_write_check_kernel<int64_t, int64_t><<<1, kWriteCheckThreads, 0, s>>>(
          slot_mapping, static_cast<const int64_t*>(block_table), bt_stride,
          static_cast<const int64_t*>(kv_len), num_seqs, mb, bl, status);
    else
      decode_write_check_kernel<int64_t, int32_t><<<1, kWriteCheckThreads, 0, s>>>(
          slot_mapping, static_cast<const int32_t*>(block_table), bt_stride,
          static_cast<const int64_t*>(kv_len), num_seqs, mb, bl, status);
  } else {
    if (bt_is_i64)
      decode_write_check_kernel<int32_t, int64_t><<<1, kWriteCheckThreads, 0, s>>>(
          slot_mapping, static_cast<const int64_t*>(block_table), bt_stride,
          static_cast<const int32_t*>(kv_len), num_seqs, mb, bl, status);
    else
      decode_write_check_kernel<int32_t, int32_t><<<1, kWriteCheckThreads, 0, s>>>(
          slot_mapping, static_cast<const int32_t*>(block_table), bt_stride,
          static_cast<const int32_t*>(kv_len), num_seqs, mb, bl, status);
  }
  return check_launch("mv_decode_write_check");
}
