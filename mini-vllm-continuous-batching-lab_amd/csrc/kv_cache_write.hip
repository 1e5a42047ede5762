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
constexpr int kSlotCountShift = 44;
constexpr uint64_t kSlotKeyMask = (uint64_t(1) << kSlotCountShift) - 1;
constexpr int kSlotsLdsMax = 4096;
constexpr int kSlotsLdsEntries = 2 * kSlotsLdsMax;  // 64 KiB of LDS
constexpr int kSlotsCheckThreads = 1024;
constexpr int kSlotsGridThreads = 256;
constexpr int64_t kSlotsMax = (int64_t(1) << (64 - kSlotCountShift)) - 1;  // count field

__device__ __forceinline__ uint32_t hash64(uint64_t k) {
  return static_cast<uint32_t>((k * 0x9E3779B97F4A7C15ull) >> 29);
}

// Inserts `key` (slot + 1); returns the number of equal keys inserted
// before it. `table` is LDS or global memory; the atomics are the
// address space's own.
template <typename Word>
__device__ __forceinline__ uint64_t count_insert(Word* table, uint32_t hmask, uint64_t key) {
  uint32_t h = hash64(key) & hmask;
  const unsigned long long first = (1ull << kSlotCountShift) | key;
  while (true) {
    const unsigned long long old = atomicCAS(reinterpret_cast<unsigned long long*>(&table[h]), 0ull, first);
    if (old == 0) return 0;
    if ((old & kSlotKeyMask) == key) {
      const unsigned long long prev =
          atomicAdd(reinterpret_cast<unsigned long long*>(&table[h]), 1ull << kSlotCountShift);
      return prev >> kSlotCountShift;
    }
    h = (h + 1) & hmask;
  }
}

__device__ __forceinline__ int32_t saturate_i32(uint64_t v) {
  return v > static_cast<uint64_t>(INT_MAX) ? INT_MAX : static_cast<int32_t>(v);
}

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

inline uint32_t pow2_at_least(int64_t v) {
  uint32_t h = 1;
  while (h < v) h <<= 1;
  return h;
}

// ---------------------------------------------------------------------------
// Fused decode + KV write precondition (mv_paged_decode_write).
//
// Phase 1 (one work group): counts the sequences whose slot is neither -1
// nor the table position of their own token kv_len - 1 (status[0]), and
// puts every other writer b -- slot s_b in block k_b at offset o_b -- into
// a hash table keyed by k_b + 1 whose value is the minimum of
// (o_b << 12) | b over the writers of that block, as 64-bit words
// ((k_b + 1) << 32) | value (0: empty). Built in LDS, then stored to the
// workspace.
// Phase 2 (a grid of (sequence c, 256 table entries)): an entry j that c
// attends (j < ceil(kv_c / bs)) whose block is in the table is counted
// (status[1]) when the block's smallest written offset lies below c's
// limit in that block, min(bs, kv_c - j bs), unless that writer is c itself
// at its own last position. That is exact: a write at offset o is read
// through entry (c, j) iff o < the limit, and if the smallest-offset writer
// is c's own last position, every other writer of the block is either not
// attended by c or writes c's very slot (a duplicate slot). Phase 2 does
// not count c's own entry in that last case; phase 1 does, once per block
// whose smallest written offset has two or more writers, so that status[1]
// is exactly the number of attended entries (c, j) through which c reads a
// slot that some writer other than c-at-its-last-entry writes.
constexpr int kWriteCheckThreads = 1024;
constexpr int kWriteCheckEntries = 2 * MV_WRITE_CHECK_MAX_SEQS;  // 64 KiB of LDS
constexpr int kWriterSeqBits = 12;  // MV_WRITE_CHECK_MAX_SEQS = 1 << 12
constexpr int kWriterMaxBlockLog2 = 20;  // offsets < 2^20 fit the value's upper bits
static_assert(kWriterMaxBlockLog2 + kWriterSeqBits <= 32, "writer value bits");
constexpr int kSharedCheckThreads = 256;
static_assert(MV_WRITE_CHECK_MAX_SEQS == (1 << kWriterSeqBits), "writer index bits");

__device__ __forceinline__ uint32_t hash32(uint32_t k) { return (k * 0x9E3779B1u) >> 7; }

// Phase 1 for one work group of kWriteCheckThreads threads (called by
// every thread): builds the writers' table in `table` (LDS, hmask + 1
// entries) and stores it to `writers`; returns, in every thread, the
// own-slot failures and the blocks whose smallest written offset has two or
// more writers. `dup_blocks` (LDS, kWriteCheckEntries / 32 words) and
// `s_red` (LDS, 2 ints) are scratch.
template <typename KV, typename BT>
__device__ __forceinline__ int2 build_writers(const int64_t* slots, const BT* bt, int64_t bt_stride,
                                              const KV* kv_len, int32_t num_seqs, int32_t max_blocks,
                                              int32_t bs_log2, uint64_t* writers, uint32_t hmask,
                                              uint64_t* table, uint32_t* dup_blocks, int* s_red) {
  constexpr int kMine = MV_WRITE_CHECK_MAX_SEQS / kWriteCheckThreads;
  for (uint32_t i = threadIdx.x; i <= hmask; i += kWriteCheckThreads) table[i] = 0;
  for (uint32_t i = threadIdx.x; i < kWriteCheckEntries / 32; i += kWriteCheckThreads) dup_blocks[i] = 0;
  if (threadIdx.x == 0) { s_red[0] = 0; s_red[1] = 0; }
  __syncthreads();
  int bad = 0;
  uint64_t mine[kMine];  // this thread's writers' words (0: none)
#pragma unroll
  for (int i = 0; i < kMine; ++i) mine[i] = 0;
#pragma unroll
  for (int i = 0; i < kMine; ++i) {
    const int b = static_cast<int>(threadIdx.x) + i * kWriteCheckThreads;
    if (b >= num_seqs) continue;
    const int64_t s = slots[b];
    if (s == -1) continue;
    const int64_t kv = static_cast<int64_t>(kv_len[b]);
    const int64_t e = (kv - 1) >> bs_log2;
    const int64_t off = (kv - 1) & ((int64_t(1) << bs_log2) - 1);
    bool ok = kv >= 1 && e < max_blocks;
    int64_t blk = -1;
    if (ok) {
      blk = static_cast<int64_t>(bt[b * bt_stride + e]);
      // ids that cannot be keyed lie far outside any pool
      ok = blk >= 0 && blk < int64_t(0xFFFFFFFF) && s == (blk << bs_log2) + off;
    }
    if (!ok) { ++bad; continue; }
    const uint64_t key = static_cast<uint64_t>(blk + 1) << 32;
    const uint64_t word = key | (static_cast<uint64_t>(off) << kWriterSeqBits) | static_cast<uint64_t>(b);
    mine[i] = word;
    uint32_t h = hash32(static_cast<uint32_t>(blk + 1)) & hmask;
    while (true) {
      const unsigned long long old = atomicCAS(reinterpret_cast<unsigned long long*>(&table[h]), 0ull,
                                               static_cast<unsigned long long>(key | 0xFFFFFFFFull));
      if (old == 0 || (old & 0xFFFFFFFF00000000ull) == key) {
        // the same key in the high bits: the word's minimum is the value's
        atomicMin(reinterpret_cast<unsigned long long*>(&table[h]), static_cast<unsigned long long>(word));
        break;
      }
      h = (h + 1) & hmask;
    }
  }
  if (bad) atomicAdd(&s_red[0], bad);
  __syncthreads();
  // A writer at its block's smallest written offset that is not the
  // block's minimum word writes the minimum writer's slot too.
  constexpr uint64_t kSeqMask = (1u << kWriterSeqBits) - 1;
#pragma unroll
  for (int i = 0; i < kMine; ++i) {
    const uint64_t word = mine[i];
    if (!word) continue;
    uint32_t h = hash32(static_cast<uint32_t>(word >> 32)) & hmask;
    while ((table[h] ^ word) >> 32) h = (h + 1) & hmask;  // present: inserted above
    const uint64_t least = table[h];
    if (((least ^ word) & 0xFFFFFFFFull) >> kWriterSeqBits == 0 && (least & kSeqMask) != (word & kSeqMask))
      atomicOr(&dup_blocks[h >> 5], 1u << (h & 31));
  }
  __syncthreads();
  int dups = 0;
  for (uint32_t i = threadIdx.x; i < kWriteCheckEntries / 32; i += kWriteCheckThreads)
    dups += __popc(dup_blocks[i]);
  if (dups) atomicAdd(&s_red[1], dups);
  for (uint32_t i = threadIdx.x; i <= hmask; i += kWriteCheckThreads) writers[i] = table[i];
  __syncthreads();
  return make_int2(s_red[0], s_red[1]);
}

template <typename KV, typename BT>
__global__ __launch_bounds__(kWriteCheckThreads) void decode_write_check_kernel(
    const int64_t* slots, const BT* bt, int64_t bt_stride, const KV* kv_len, int32_t num_seqs,
    int32_t max_blocks, int32_t bs_log2, uint64_t* writers, uint32_t hmask, int32_t* status) {
  __shared__ uint64_t table[kWriteCheckEntries];
  __shared__ uint32_t dup_blocks[kWriteCheckEntries / 32];
  __shared__ int s_red[2];
  const int2 r = build_writers(slots, bt, bt_stride, kv_len, num_seqs, max_blocks, bs_log2, writers,
                               hmask, table, dup_blocks, s_red);
  if (threadIdx.x == 0) {
    status[MV_WRITE_CHECK_OWN_SLOT] = r.x;
    status[MV_WRITE_CHECK_SHARED] = r.y;
  }
}

// The fused decode step's checks in one work group (mv_decode_step_check):
// the slot check of the step's decode slots (as slots_check_lds_kernel),
// phase 1 of the fused-write check (build_writers), the positions check
// and the gather of the rotary tables' rows at each position (clamped into
// the tables; out-of-range positions are counted).
struct StepCheckArgs {
  const int64_t* slots;
  const void* bt;
  const void* kv_len;
  const int64_t* positions;  // null: no positions check, no rows
  const char* cos;
  const char* sin;
  char* cos_rows;
  char* sin_rows;
  uint64_t* writers;
  int32_t* status;  // MV_STEP_* words
  int64_t bt_stride, total_slots, max_positions, table_stride;  // table_stride in bytes
  int32_t num_seqs, max_blocks, bs_log2, row_bytes;
  uint32_t slot_hmask, writer_hmask;
};

template <typename KV, typename BT>
__global__ __launch_bounds__(kWriteCheckThreads) void decode_step_check_kernel(StepCheckArgs a) {
  __shared__ uint64_t slot_table[kSlotsLdsEntries];
  __shared__ uint64_t table[kWriteCheckEntries];
  __shared__ uint32_t dup_blocks[kWriteCheckEntries / 32];
  __shared__ int s_red[2];
  __shared__ int s_bad, s_pos_bad;
  __shared__ unsigned long long s_pairs;
  for (uint32_t i = threadIdx.x; i <= a.slot_hmask; i += kWriteCheckThreads) slot_table[i] = 0;
  if (threadIdx.x == 0) { s_bad = 0; s_pairs = 0; s_pos_bad = 0; }
  // rotary rows: chunk i of 16 bytes of row b of table tb (the loads of
  // every chunk go out before any other work waits on memory)
  int pos_bad = 0;
  if (a.positions) {
    const int cpr = a.row_bytes / 16;
    const int n = 2 * a.num_seqs * cpr;
    for (int i = threadIdx.x; i < n; i += kWriteCheckThreads) {
      const int tb = i / (a.num_seqs * cpr);
      const int r = i - tb * a.num_seqs * cpr;
      const int b = r / cpr, c = r - b * cpr;
      const int64_t p = a.positions[b];
      if (tb == 0 && c == 0) pos_bad += p < 0 || p >= a.max_positions;
      const int64_t row = p < 0 ? 0 : (p >= a.max_positions ? a.max_positions - 1 : p);
      const uint4 v = *reinterpret_cast<const uint4*>((tb ? a.sin : a.cos) + row * a.table_stride + c * 16);
      *reinterpret_cast<uint4*>((tb ? a.sin_rows : a.cos_rows) + static_cast<int64_t>(b) * a.row_bytes + c * 16) = v;
    }
  }
  __syncthreads();
  int bad = 0;
  uint64_t pairs = 0;
  for (int x = threadIdx.x; x < a.num_seqs; x += kWriteCheckThreads) {
    const int64_t s = a.slots[x];
    if (s == -1) continue;
    if (s < 0 || s >= a.total_slots) { ++bad; continue; }
    pairs += count_insert(slot_table, a.slot_hmask, static_cast<uint64_t>(s) + 1);
  }
  if (bad) atomicAdd(&s_bad, bad);
  if (pairs) atomicAdd(&s_pairs, static_cast<unsigned long long>(pairs));
  if (pos_bad) atomicAdd(&s_pos_bad, pos_bad);
  const int2 r = build_writers(a.slots, static_cast<const BT*>(a.bt), a.bt_stride,
                               static_cast<const KV*>(a.kv_len), a.num_seqs, a.max_blocks, a.bs_log2,
                               a.writers, a.writer_hmask, table, dup_blocks, s_red);
  if (threadIdx.x == 0) {  // build_writers ends on a barrier: the counts are complete
    a.status[MV_STEP_SLOTS_OUT_OF_RANGE] = s_bad;
    a.status[MV_STEP_SLOTS_DUPLICATES] = saturate_i32(s_pairs);
    a.status[MV_STEP_WRITE_OWN_SLOT] = r.x;
    a.status[MV_STEP_WRITE_SHARED] = r.y;
    a.status[MV_STEP_POSITIONS] = s_pos_bad;
  }
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
  static_assert(MV_STEP_WRITE_SHARED - MV_STEP_WRITE_OWN_SLOT ==
                    MV_WRITE_CHECK_SHARED - MV_WRITE_CHECK_OWN_SLOT,
                "phase 2 adds to the step's shared-read word");
  if (!status) return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_step_check: null status");
  if (num_seqs < 0 || max_blocks < 0 || num_blocks < 0)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_step_check: negative size");
  if (num_seqs > MV_WRITE_CHECK_MAX_SEQS)
    return fail(MV_ERR_UNSUPPORTED, "mv_decode_step_check: %d sequences (at most %d)", num_seqs,
                MV_WRITE_CHECK_MAX_SEQS);
  if (!is_pow2(block_size) || ilog2_exact(block_size) > kWriterMaxBlockLog2)
    return fail(MV_ERR_UNSUPPORTED,
                "mv_decode_step_check: block_size %d is not a power of 2 up to 2^%d", block_size,
                kWriterMaxBlockLog2);
  const int64_t total_slots = num_blocks * block_size;
  if (total_slots >= static_cast<int64_t>(kSlotKeyMask))
    return fail(MV_ERR_UNSUPPORTED, "mv_decode_step_check: %lld slots in the pool (fewer than 2^44)",
                (long long)total_slots);
  if (num_seqs > 0 && (!slot_mapping || !kv_len || (max_blocks > 0 && !block_table)))
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_step_check: null pointer");
  const int eb = dtype_bytes(dtype);
  if (positions) {
    if (eb == 0 || head_dim <= 0 || (head_dim * eb) % 16 || max_positions <= 0 || !cos_table ||
        !sin_table || !cos_rows || !sin_rows)
      return fail(MV_ERR_INVALID_ARGUMENT,
                  "mv_decode_step_check: rotary rows need the tables, the rows, a dtype and a "
                  "head_dim of whole 16-byte pieces");
    const uintptr_t al = reinterpret_cast<uintptr_t>(cos_table) | reinterpret_cast<uintptr_t>(sin_table) |
                         reinterpret_cast<uintptr_t>(cos_rows) | reinterpret_cast<uintptr_t>(sin_rows) |
                         static_cast<uintptr_t>(table_stride * eb);
    if (al % 16)
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_step_check: rotary tables or rows not 16-byte aligned");
    if (table_stride < head_dim)
      return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_step_check: table stride %lld < head_dim %d",
                  (long long)table_stride, head_dim);
  }
  const size_t need = mv_decode_write_check_workspace_bytes(num_seqs);
  if (!workspace || workspace_bytes < need)
    return fail(MV_ERR_INVALID_ARGUMENT,
                "mv_decode_step_check: %d sequences need a %zu-byte workspace (got %zu)", num_seqs,
                need, workspace ? workspace_bytes : size_t(0));
  if (reinterpret_cast<uintptr_t>(workspace) % 8)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_step_check: workspace not 8-byte aligned");
  const int mb = block_table ? max_blocks : 0;
  const unsigned chunks = static_cast<unsigned>((mb + kSharedCheckThreads - 1) / kSharedCheckThreads);
  if (chunks > 65535)
    return fail(MV_ERR_INVALID_ARGUMENT, "mv_decode_step_check: %d table columns is too many", mb);
  StepCheckArgs a;
  a.slots = slot_mapping;
  a.bt = block_table;
  a.kv_len = kv_len;
  a.positions = positions;
  a.cos = static_cast<const char*>(cos_table);
  a.sin = static_cast<const char*>(sin_table);
  a.cos_rows = static_cast<char*>(cos_rows);
  a.sin_rows = static_cast<char*>(sin_rows);
  a.writers = static_cast<uint64_t*>(workspace);
  a.status = status;
  a.bt_stride = bt_stride;
  a.total_slots = total_slots;
  a.max_positions = max_positions;
  a.table_stride = table_stride * eb;
  a.num_seqs = num_seqs;
  a.max_blocks = mb;
  a.bs_log2 = ilog2_exact(block_size);
  a.row_bytes = head_dim * eb;
  a.slot_hmask = pow2_at_least(std::max<int64_t>(64, 2 * int64_t(num_seqs))) - 1;
  a.writer_hmask = static_cast<uint32_t>(need / sizeof(uint64_t)) - 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(num_seqs), chunks);
  const bool scan = num_seqs > 0 && chunks > 0;
#define MV_STEP_CHECK(KV, BT)                                                                     \
  do {                                                                                            \
    decode_step_check_kernel<KV, BT><<<1, kWriteCheckThreads, 0, s>>>(a);                         \
    if (scan)                                                                                     \
      decode_shared_slot_kernel<KV, BT><<<grid, kSharedCheckThreads, 0, s>>>(                     \
          static_cast<const BT*>(block_table), bt_stride, static_cast<const KV*>(kv_len), mb,      \
          a.bs_log2, a.writers, a.writer_hmask, status + MV_STEP_WRITE_OWN_SLOT);                 \
  } while (0)
  if (kv_len_is_i64) {
    if (bt_is_i64) MV_STEP_CHECK(int64_t, int64_t);
    else MV_STEP_CHECK(int64_t, int32_t);
  } else {
    if (bt_is_i64) MV_STEP_CHECK(int32_t, int64_t);
    else MV_STEP_CHECK(int32_t, int32_t);
  }
#undef MV_STEP_CHECK
  return check_launch("mv_decode_step_check");
}
