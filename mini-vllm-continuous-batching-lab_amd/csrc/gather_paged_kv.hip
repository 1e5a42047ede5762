// Gather of cached prefix K/V into contiguous rows (prefill support).
//
// Replaces the Triton `_gather_prefix_kv_kernel`
// (mini_vllm/attention/paged_attention_gpu.py:330-388) and follows
// `gather_paged_kv` (mini_vllm/cache/cache_read.py:19-84): for sequence i,
// token pos < cu_tokens[i+1] - cu_tokens[i] of table row seq_rows[i]
//   out[cu_tokens[i] + pos, h, :] = cache[bt[row, pos / BS], h, pos % BS, :]
// The flat token -> sequence map is a binary search over cu_tokens, so the
// host builds no per-token index arrays. Each thread moves one 16-byte
// chunk (head_dim * element bytes is a multiple of 16 for every supported
// shape; the host checks).
#include <algorithm>

#include "mv_common.h"

namespace mv {
namespace {

struct GatherArgs {
  const char* key_cache;
  const char* value_cache;
  const void* block_table;
  int64_t bt_stride;
  const int64_t* seq_rows;
  const int64_t* cu_tokens;  // [num_seqs + 1]
  int32_t num_seqs;
  int64_t total_tokens;
  char* out_key;
  char* out_value;
  int32_t num_kv_heads, row_bytes, bs_log2;
  int64_t num_blocks;
};

template <typename BT>
__global__ __launch_bounds__(256) void gather_paged_kv_kernel(GatherArgs a) {
  const int chunks = a.row_bytes / 16;
  const int64_t per_tensor = a.total_tokens * a.num_kv_heads * chunks;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < 2 * per_tensor;
       i += (int64_t)gridDim.x * blockDim.x) {
    const bool is_v = i >= per_tensor;
    const int64_t r = is_v ? i - per_tensor : i;
    const int64_t row = r / chunks;
    const int chunk = static_cast<int>(r - row * chunks);
    const int64_t tok = row / a.num_kv_heads;
    const int h = static_cast<int>(row - tok * a.num_kv_heads);
    // last sequence with cu_tokens[s] <= tok
    int lo = 0, hi = a.num_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.cu_tokens[mid] <= tok) lo = mid; else hi = mid - 1;
    }
    const int64_t pos = tok - a.cu_tokens[lo];
    const BT* bt_row = static_cast<const BT*>(a.block_table) + a.seq_rows[lo] * a.bt_stride;
    const int64_t blk = static_cast<int64_t>(bt_row[pos >> a.bs_log2]);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (blk >= 0 && blk < a.num_blocks) {
      const int64_t src_row = ((blk * a.num_kv_heads + h) << a.bs_log2) + (pos & ((1 << a.bs_log2) - 1));
      v = reinterpret_cast<const uint4*>((is_v ? a.value_cache : a.key_cache) + src_row * a.row_bytes)[chunk];
    }
    reinterpret_cast<uint4*>((is_v ? a.out_value : a.out_key) + row * a.row_bytes)[chunk] = v;
  }
}

}  // namespace
}  // namespace mv

extern "C" int mv_gather_paged_kv(const void* key_cache, const void* value_cache,
                                  const void* block_table, int32_t bt_is_i64, int64_t bt_stride,
                                  const int64_t* seq_rows, const int64_t* cu_tokens,
                                  int32_t num_seqs, int64_t total_tokens, void* out_key,
                                  void* out_value, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t block_size, int64_t num_blocks, int32_t dtype,
                                  void* stream) {
  using namespace mv;
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(MV_ERR_UNSUPPORTED, "mv_gather_paged_kv: unknown dtype %d", dtype);
  if (!is_pow2(block_size))
    return fail(MV_ERR_UNSUPPORTED, "mv_gather_paged_kv: block_size %d is not a power of 2", block_size);
  if (num_seqs < 0 || total_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_gather_paged_kv: bad sizes");
  if (total_tokens == 0 || num_seqs == 0) return MV_OK;
  const int row_bytes = head_dim * eb;
  if (row_bytes % 16)
    return fail(MV_ERR_UNSUPPORTED, "mv_gather_paged_kv: head_dim*elem bytes %d not a multiple of 16",
                row_bytes);
  if (!key_cache || !value_cache || !block_table || !seq_rows || !cu_tokens || !out_key || !out_value)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_gather_paged_kv: null pointer");
  if ((reinterpret_cast<uintptr_t>(key_cache) | reinterpret_cast<uintptr_t>(value_cache) |
       reinterpret_cast<uintptr_t>(out_key) | reinterpret_cast<uintptr_t>(out_value)) % 16)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_gather_paged_kv: buffers not 16-byte aligned");
  GatherArgs a;
  a.key_cache = static_cast<const char*>(key_cache);
  a.value_cache = static_cast<const char*>(value_cache);
  a.block_table = block_table;
  a.bt_stride = bt_stride;
  a.seq_rows = seq_rows;
  a.cu_tokens = cu_tokens;
  a.num_seqs = num_seqs;
  a.total_tokens = total_tokens;
  a.out_key = static_cast<char*>(out_key);
  a.out_value = static_cast<char*>(out_value);
  a.num_kv_heads = num_kv_heads;
  a.row_bytes = row_bytes;
  a.bs_log2 = ilog2_exact(block_size);
  a.num_blocks = num_blocks;
  const int64_t work = 2 * total_tokens * num_kv_heads * (row_bytes / 16);
  const int64_t blocks = std::min<int64_t>((work + 255) / 256, 65536);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (bt_is_i64) gather_paged_kv_kernel<int64_t><<<blocks, 256, 0, s>>>(a);
  else gather_paged_kv_kernel<int32_t><<<blocks, 256, 0, s>>>(a);
  return check_launch("mv_gather_paged_kv");
}
