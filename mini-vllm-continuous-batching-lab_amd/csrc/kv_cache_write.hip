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
#include "mv_step_check.h"

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

// ---------------------------------------------------------------------------
// Slot check: out-of-range slots and duplicate pairs in O(T) expected work.
//
// Every in-range slot is inserted into an open-addressing hash table of
// 64-bit words (count << 44) | (slot + 1), 0 marking an empty entry. An
// insert that finds its slot already present adds one to the count and
// learns how many equal slots were inserted before it; summed over all
// inserts that is sum_v k_v (k_v - 1) / 2 = the number of pairs (x < y)
// with slots[x] == slots[y], whatever the insertion order. The table has at
// least twice as many entries as slots, so every probe sequence ends.
// Up to kSlotsLdsMax slots one work group does it in LDS; beyond, a grid
// does it in a workspace table cleared by a fill kernel first.
constexpr int kSlotsLdsMax = 4096;
constexpr int kSlotsLdsEntries = 2 * kSlotsLdsMax;  // 64 KiB of LDS
constexpr int kSlotsCheckThreads = 1024;
constexpr int kSlotsGridThreads = 256;
constexpr int64_t kSlotsMax = (int64_t(1) << (64 - kSlotCountShift)) - 1;  // count field

__global__ __launch_bounds__(kSlotsCheckThreads) void slots_check_lds_kernel(
    const int64_t* slots, int32_t n, int64_t total_slots, uint32_t hmask, int32_t* status) {
  __shared__ uint64_t table[kSlotsLdsEntries];
  __shared__ int s_bad;
  __shared__ unsigned long long s_pairs;
  for (uint32_t i = threadIdx.x; i <= hmask; i += kSlotsCheckThreads) table[i] = 0;
  if (threadIdx.x == 0) { s_bad = 0; s_pairs = 0; }
  __syncthreads();
  int bad = 0;
  uint64_t pairs = 0;
  for (int x = threadIdx.x; x < n; x += kSlotsCheckThreads) {
    const int64_t s = slots[x];
    if (s == -1) continue;
    if (s < 0 || s >= total_slots) { ++bad; continue; }
    pairs += count_insert(table, hmask, static_cast<uint64_t>(s) + 1);
  }
  if (bad) atomicAdd(&s_bad, bad);
  if (pairs) atomicAdd(&s_pairs, static_cast<unsigned long long>(pairs));
  __syncthreads();
  if (threadIdx.x == 0) {
    status[MV_SLOTS_OUT_OF_RANGE] = s_bad;
    status[MV_SLOTS_DUPLICATES] = saturate_i32(s_pairs);
  }
}

__global__ __launch_bounds__(kSlotsGridThreads) void slots_clear_kernel(uint64_t* table,
                                                                        int64_t entries,
                                                                        int32_t* status) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kSlotsGridThreads;
  for (int64_t i = blockIdx.x * int64_t(kSlotsGridThreads) + threadIdx.x; i < entries; i += stride)
    table[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x < 2) status[threadIdx.x] = 0;
}

__global__ __launch_bounds__(kSlotsGridThreads) void slots_check_grid_kernel(
    const int64_t* slots, int64_t n, int64_t total_slots, uint64_t* table, uint32_t hmask,
    int32_t* status) {
  __shared__ int s_bad;
  __shared__ unsigned long long s_pairs;
  if (threadIdx.x == 0) { s_bad = 0; s_pairs = 0; }
  __syncthreads();
  const int64_t x = blockIdx.x * int64_t(kSlotsGridThreads) + threadIdx.x;
  if (x < n) {
    const int64_t s = slots[x];
    if (s != -1) {
      if (s < 0 || s >= total_slots) {
        atomicAdd(&s_bad, 1);
      } else {
        const uint64_t prev = count_insert(table, hmask, static_cast<uint64_t>(s) + 1);
        if (prev) atomicAdd(&s_pairs, static_cast<unsigned long long>(prev));
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    if (s_bad) atomicAdd(&status[MV_SLOTS_OUT_OF_RANGE], s_bad);
    if (s_pairs) {  // saturating add
      int32_t* p = &status[MV_SLOTS_DUPLICATES];
      int32_t old = *p;
      while (true) {
        const int32_t want = saturate_i32(static_cast<uint64_t>(old) + s_pairs);
        const int32_t seen = atomicCAS(p, old, want);
        if (seen == old) break;
        old = seen;
      }
    }
  }
}

// The fused-write precondition (phases 1 and 2) and the step check are
// described, and phase 1 and the step check's body defined, in
// mv_step_check.h (the decode plan's one-launch form runs the step check
// too).

template <typename KV, typename BT>
__global__ __launch_bounds__(kWriteCheckThreads) void decode_write_check_kernel(
    const int64_t* slots, const BT* bt, int64_t bt_stride, const KV* kv_len, int32_t num_seqs,
    int32_t max_blocks, int32_t bs_log2, uint64_t* writers, uint32_t hmask, int32_t* status) {
  __shared__ uint64_t table[kWriteCheckEntries];
  __shared__ uint32_t dup_blocks[kWriteCheckEntries / 32];
  __shared__ int s_red[2];
  const int2 r = build_writers<kWriteCheckThreads, MV_WRITE_CHECK_MAX_SEQS>(
      slots, bt, bt_stride, kv_len, num_seqs, max_blocks, bs_log2, writers, hmask, table, dup_blocks, s_red);
  if (threadIdx.x == 0) {
    status[MV_WRITE_CHECK_OWN_SLOT] = r.x;
    status[MV_WRITE_CHECK_SHARED] = r.y;
  }
}

template <typename KV, typename BT>
__global__ __launch_bounds__(kWriteCheckThreads) void decode_step_check_kernel(StepCheckArgs a) {
  __shared__ uint64_t slot_table[kSlotsLdsEntries];
  __shared__ uint64_t table[kWriteCheckEntries];
  __shared__ uint32_t dup_blocks[kWriteCheckEntries / 32];
  __shared__ int s_red[2];
  __shared__ int s_cnt[2];
  __shared__ unsigned long long s_pairs;
  step_check_body<KV, BT, kWriteCheckThreads, MV_WRITE_CHECK_MAX_SEQS>(a, slot_table, table, dup_blocks, s_red,
                                                                       s_cnt, &s_pairs);
}

template <typename KV, typename BT>
__global__ __launch_bounds__(kSharedCheckThreads) void decode_shared_slot_kernel(
    const BT* bt, int64_t bt_stride, const KV* kv_len, int32_t max_blocks, int32_t bs_log2,
    const uint64_t* writers, uint32_t hmask, int32_t* status) {
  const int c = blockIdx.x;
  const int64_t j = static_cast<int64_t>(blockIdx.y) * kSharedCheckThreads + threadIdx.x;
  // the table entry is loaded beside the length (j < max_blocks: in the row)
  const int64_t blk = j < max_blocks ? static_cast<int64_t>(bt[c * bt_stride + j]) : -1;
  const int64_t kv = static_cast<int64_t>(kv_len[c]);
  if (kv < 1) return;  // reported by the decode plan
  const int64_t bs = int64_t(1) << bs_log2;
  const int64_t n = min<int64_t>((kv + bs - 1) >> bs_log2, max_blocks);
  if (static_cast<int64_t>(blockIdx.y) * kSharedCheckThreads >= n) return;
  int hit = 0;
  if (j < n) {
    if (blk >= 0 && blk < int64_t(0xFFFFFFFF)) {
      const uint64_t key = static_cast<uint64_t>(blk + 1) << 32;
      uint32_t h = hash32(static_cast<uint32_t>(blk + 1)) & hmask;
      while (true) {
        const uint64_t w = writers[h];
        if (w == 0) break;
        if ((w & 0xFFFFFFFF00000000ull) == key) {
          const int b = static_cast<int>(w & ((1u << kWriterSeqBits) - 1));
          const int64_t off = static_cast<int64_t>((w & 0xFFFFFFFFull) >> kWriterSeqBits);
          const int64_t lim = min<int64_t>(bs, kv - (j << bs_log2));
          hit = off < lim && !(b == c && j == ((kv - 1) >> bs_log2));
          break;
        }
        h = (h + 1) & hmask;
      }
    }
  }
  __shared__ int s_hits;
  if (threadIdx.x == 0) s_hits = 0;
  __syncthreads();
  if (hit) atomicAdd(&s_hits, 1);
  __syncthreads();
  if (threadIdx.x == 0 && s_hits) atomicAdd(&status[MV_WRITE_CHECK_SHARED], s_hits);
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

extern "C" size_t mv_kv_slots_check_workspace_bytes(int64_t num_tokens) {
  using namespace mv;
  if (num_tokens <= kSlotsLdsMax) return 0;
  return static_cast<size_t>(pow2_at_least(2 * num_tokens)) * sizeof(uint64_t);
}

extern "C" int mv_kv_slots_check(const int64_t* slot_mapping, int64_t num_tokens,
                                 int64_t total_slots, int32_t* status, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  using namespace mv;
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_slots_check: null status");
  if (num_tokens < 0 || total_slots < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_slots_check: negative size");
  if (num_tokens > kSlotsMax)
    return fail(MV_ERR_UNSUPPORTED, "mv_kv_slots_check: %lld tokens (at most %lld)",
                (long long)num_tokens, (long long)kSlotsMax);
  if (total_slots >= static_cast<int64_t>(kSlotKeyMask))
    return fail(MV_ERR_UNSUPPORTED, "mv_kv_slots_check: %lld slots in the pool (fewer than 2^44)",
                (long long)total_slots);
  if (num_tokens > 0 && !slot_mapping)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_slots_check: null slots");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (num_tokens <= kSlotsLdsMax) {
    const uint32_t entries = pow2_at_least(std::max<int64_t>(64, 2 * num_tokens));
    slots_check_lds_kernel<<<1, kSlotsCheckThreads, 0, s>>>(
        slot_mapping, static_cast<int32_t>(num_tokens), total_slots, entries - 1, status);
    return check_launch("mv_kv_slots_check");
  }
  const size_t need = mv_kv_slots_check_workspace_bytes(num_tokens);
  if (!workspace || workspace_bytes < need)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_kv_slots_check: %lld tokens need a %zu-byte workspace (got %zu)",
                (long long)num_tokens, need, workspace ? workspace_bytes : size_t(0));
  if (reinterpret_cast<uintptr_t>(workspace) % 8)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_kv_slots_check: workspace not 8-byte aligned");
  uint64_t* table = static_cast<uint64_t*>(workspace);
  const int64_t entries = static_cast<int64_t>(need / sizeof(uint64_t));
  const int64_t clear_groups = std::min<int64_t>((entries + kSlotsGridThreads - 1) / kSlotsGridThreads, 1024);
  slots_clear_kernel<<<static_cast<unsigned>(clear_groups), kSlotsGridThreads, 0, s>>>(table, entries,
                                                                                     status);
  const int64_t groups = (num_tokens + kSlotsGridThreads - 1) / kSlotsGridThreads;
  slots_check_grid_kernel<<<static_cast<unsigned>(groups), kSlotsGridThreads, 0, s>>>(
      slot_mapping, num_tokens, total_slots, table, static_cast<uint32_t>(entries - 1), status);
  return check_launch("mv_kv_slots_check");
}

extern "C" size_t mv_decode_write_check_workspace_bytes(int32_t num_seqs) {
  using namespace mv;
  if (num_seqs < 0 || num_seqs > MV_WRITE_CHECK_MAX_SEQS) return 0;
  return static_cast<size_t>(pow2_at_least(std::max<int64_t>(64, 2 * int64_t(num_seqs)))) *
         sizeof(uint64_t);
}

extern "C" int mv_decode_write_check(const int64_t* slot_mapping, const void* block_table,
                                     int32_t bt_is_i64, int64_t bt_stride, const void* kv_len,
                                     int32_t kv_len_is_i64, int32_t num_seqs, int32_t max_blocks,
                                     int32_t block_size, int32_t* status, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  using namespace mv;
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_write_check: null status");
  if (num_seqs < 0 || max_blocks < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_write_check: negative size");
  if (num_seqs > MV_WRITE_CHECK_MAX_SEQS)
    return fail(MV_ERR_UNSUPPORTED, "mv_decode_write_check: %d sequences (at most %d)", num_seqs,
                MV_WRITE_CHECK_MAX_SEQS);
  if (!is_pow2(block_size) || ilog2_exact(block_size) > kWriterMaxBlockLog2)
    return fail(MV_ERR_UNSUPPORTED,
                "mv_decode_write_check: block_size %d is not a power of 2 up to 2^%d", block_size,
                kWriterMaxBlockLog2);
  if (num_seqs > 0 && (!slot_mapping || !kv_len || (max_blocks > 0 && !block_table)))
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_write_check: null pointer");
  const size_t need = mv_decode_write_check_workspace_bytes(num_seqs);
  if (!workspace || workspace_bytes < need)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_decode_write_check: %d sequences need a %zu-byte workspace (got %zu)",
                num_seqs, need, workspace ? workspace_bytes : size_t(0));
  if (reinterpret_cast<uintptr_t>(workspace) % 8)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_write_check: workspace not 8-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int bl = ilog2_exact(block_size);
  const int mb = block_table ? max_blocks : 0;
  uint64_t* writers = static_cast<uint64_t*>(workspace);
  const uint32_t hmask = static_cast<uint32_t>(need / sizeof(uint64_t)) - 1;
  const unsigned chunks = static_cast<unsigned>((mb + kSharedCheckThreads - 1) / kSharedCheckThreads);
  if (chunks > 65535)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_write_check: %d table columns is too many", mb);
  const dim3 grid(static_cast<unsigned>(num_seqs), chunks);
  const bool scan = num_seqs > 0 && chunks > 0;
#define MV_WRITE_CHECK(KV, BT)                                                                   \
  do {                                                                                           \
    decode_write_check_kernel<KV, BT><<<1, kWriteCheckThreads, 0, s>>>(                          \
        slot_mapping, static_cast<const BT*>(block_table), bt_stride,                            \
        static_cast<const KV*>(kv_len), num_seqs, mb, bl, writers, hmask, status);               \
    if (scan)                                                                                    \
      decode_shared_slot_kernel<KV, BT><<<grid, kSharedCheckThreads, 0, s>>>(                    \
          static_cast<const BT*>(block_table), bt_stride, static_cast<const KV*>(kv_len), mb, bl, \
          writers, hmask, status);                                                               \
  } while (0)
  if (kv_len_is_i64) {
    if (bt_is_i64) MV_WRITE_CHECK(int64_t, int64_t);
    else MV_WRITE_CHECK(int64_t, int32_t);
  } else {
    if (bt_is_i64) MV_WRITE_CHECK(int32_t, int64_t);
    else MV_WRITE_CHECK(int32_t, int32_t);
  }
#undef MV_WRITE_CHECK
  return check_launch("mv_decode_write_check");
}

namespace mv {

int step_check_prepare(const char* who, const int64_t* slot_mapping, const void* block_table,
                       int64_t bt_stride, const void* kv_len, int32_t num_seqs, int32_t max_blocks,
                       int32_t block_size, int64_t num_blocks, const int64_t* positions,
                       const void* cos_table, const void* sin_table, int64_t table_stride,
                       int64_t max_positions, int32_t head_dim, int32_t dtype, void* cos_rows,
                       void* sin_rows, int32_t* status, void* workspace, size_t workspace_bytes,
                       StepCheckArgs* a) {
  static_assert(MV_STEP_WRITE_SHARED - MV_STEP_WRITE_OWN_SLOT ==
                    MV_WRITE_CHECK_SHARED - MV_WRITE_CHECK_OWN_SLOT,
                "phase 2 adds to the step's shared-read word");
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "%s: null status", who);
  if (num_seqs < 0 || max_blocks < 0 || num_blocks < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: negative size", who);
  if (num_seqs > MV_WRITE_CHECK_MAX_SEQS)
    return fail(MV_ERR_UNSUPPORTED, "%s: %d sequences (at most %d)", who, num_seqs, MV_WRITE_CHECK_MAX_SEQS);
  if (!is_pow2(block_size) || ilog2_exact(block_size) > kWriterMaxBlockLog2)
    return fail(MV_ERR_UNSUPPORTED, "%s: block_size %d is not a power of 2 up to 2^%d", who, block_size,
                kWriterMaxBlockLog2);
  const int64_t total_slots = num_blocks * block_size;
  if (total_slots >= static_cast<int64_t>(kSlotKeyMask))
    return fail(MV_ERR_UNSUPPORTED, "%s: %lld slots in the pool (fewer than 2^44)", who,
                (long long)total_slots);
  if (num_seqs > 0 && (!slot_mapping || !kv_len || (max_blocks > 0 && !block_table)))
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: null pointer", who);
  const int eb = dtype_bytes(dtype);
  if (positions) {
    if (eb == 0 || head_dim <= 0 || (head_dim * eb) % 16 || max_positions <= 0 || !cos_table ||
        !sin_table || !cos_rows || !sin_rows)
      return fail(MV_ERR_INVALID_ARGUMENT,
                  "%s: rotary rows need the tables, the rows, a dtype and a head_dim of whole "
                  "16-byte pieces", who);
    const uintptr_t al = reinterpret_cast<uintptr_t>(cos_table) | reinterpret_cast<uintptr_t>(sin_table) |
                         reinterpret_cast<uintptr_t>(cos_rows) | reinterpret_cast<uintptr_t>(sin_rows) |
                         static_cast<uintptr_t>(table_stride * eb);
    if (al % 16) return fail(MV_ERR_INVALID_ARGUMENT, "%s: rotary tables or rows not 16-byte aligned", who);
    if (table_stride < head_dim)
      return fail(MV_ERR_INVALID_ARGUMENT, "%s: table stride %lld < head_dim %d", who,
                  (long long)table_stride, head_dim);
  }
  const size_t need = mv_decode_write_check_workspace_bytes(num_seqs);
  if (!workspace || workspace_bytes < need)
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: %d sequences need a %zu-byte workspace (got %zu)", who,
                num_seqs, need, workspace ? workspace_bytes : size_t(0));
  if (reinterpret_cast<uintptr_t>(workspace) % 8)
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: workspace not 8-byte aligned", who);
  const int mb = block_table ? max_blocks : 0;
  if ((mb + kSharedCheckThreads - 1) / kSharedCheckThreads > 65535)
    return fail(MV_ERR_INVALID_ARGUMENT, "%s: %d table columns is too many", who, mb);
  a->slots = slot_mapping;
  a->bt = block_table;
  a->kv_len = kv_len;
  a->positions = positions;
  a->cos = static_cast<const char*>(cos_table);
  a->sin = static_cast<const char*>(sin_table);
  a->cos_rows = static_cast<char*>(cos_rows);
  a->sin_rows = static_cast<char*>(sin_rows);
  a->writers = static_cast<uint64_t*>(workspace);
  a->status = status;
  a->bt_stride = bt_stride;
  a->total_slots = total_slots;
  a->max_positions = max_positions;
  a->table_stride = table_stride * eb;
  a->num_seqs = num_seqs;
  a->max_blocks = mb;
  a->bs_log2 = ilog2_exact(block_size);
  a->row_bytes = head_dim * eb;
  a->slot_hmask = pow2_at_least(std::max<int64_t>(64, 2 * int64_t(num_seqs))) - 1;
  a->writer_hmask = static_cast<uint32_t>(need / sizeof(uint64_t)) - 1;
  return MV_OK;
}

int step_check_scan(const StepCheckArgs& a, int32_t bt_is_i64, int32_t kv_len_is_i64, hipStream_t s) {
  const unsigned chunks = static_cast<unsigned>((a.max_blocks + kSharedCheckThreads - 1) / kSharedCheckThreads);
  if (a.num_seqs == 0 || chunks == 0) return MV_OK;
  const dim3 grid(static_cast<unsigned>(a.num_seqs), chunks);
#define MV_SCAN(KV, BT)                                                                              \
  decode_shared_slot_kernel<KV, BT><<<grid, kSharedCheckThreads, 0, s>>>(                            \
      static_cast<const BT*>(a.bt), a.bt_stride, static_cast<const KV*>(a.kv_len), a.max_blocks,    \
      a.bs_log2, a.writers, a.writer_hmask, a.status + MV_STEP_WRITE_OWN_SLOT)
  if (kv_len_is_i64) {
    if (bt_is_i64) MV_SCAN(int64_t, int64_t);
    else MV_SCAN(int64_t, int32_t);
  } else {
    if (bt_is_i64) MV_SCAN(int32_t, int64_t);
    else MV_SCAN(int32_t, int32_t);
  }
#undef MV_SCAN
  return MV_OK;
}

int step_check_launch(const StepCheckArgs& a, int32_t bt_is_i64, int32_t kv_len_is_i64, hipStream_t s) {
  if (kv_len_is_i64) {
    if (bt_is_i64) decode_step_check_kernel<int64_t, int64_t><<<1, kWriteCheckThreads, 0, s>>>(a);
    else decode_step_check_kernel<int64_t, int32_t><<<1, kWriteCheckThreads, 0, s>>>(a);
  } else {
    if (bt_is_i64) decode_step_check_kernel<int32_t, int64_t><<<1, kWriteCheckThreads, 0, s>>>(a);
    else decode_step_check_kernel<int32_t, int32_t><<<1, kWriteCheckThreads, 0, s>>>(a);
  }
  return step_check_scan(a, bt_is_i64, kv_len_is_i64, s);
}

}  // namespace mv

extern "C" int mv_decode_step_check(const int64_t* slot_mapping, const void* block_table,
                                    int32_t bt_is_i64, int64_t bt_stride, const void* kv_len,
                                    int32_t kv_len_is_i64, int32_t num_seqs, int32_t max_blocks,
                                    int32_t block_size, int64_t num_blocks,
                                    const int64_t* positions, const void* cos_table,
                                    const void* sin_table, int64_t table_stride,
                                    int64_t max_positions, int32_t head_dim, int32_t dtype,
                                    void* cos_rows, void* sin_rows, int32_t* status,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  using namespace mv;
  StepCheckArgs a;
  if (const int rc = step_check_prepare("mv_decode_step_check", slot_mapping, block_table, bt_stride, kv_len,
                                        num_seqs, max_blocks, block_size, num_blocks, positions, cos_table,
                                        sin_table, table_stride, max_positions, head_dim, dtype, cos_rows,
                                        sin_rows, status, workspace, workspace_bytes, &a))
    return rc;
  step_check_launch(a, bt_is_i64, kv_len_is_i64, static_cast<hipStream_t>(stream));
  return check_launch("mv_decode_step_check");
}
