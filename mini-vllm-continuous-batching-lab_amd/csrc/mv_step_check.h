// The decode step's metadata checks, shared by kv_cache_write.hip (the slot
// check, mv_decode_write_check, mv_decode_step_check) and paged_decode.hip
// (whose one-launch plan runs the step check in one of its work groups).
//
// Slot check: out-of-range slots and duplicate pairs in O(T) expected work.
// Every in-range slot is inserted into an open-addressing hash table of
// 64-bit words (count << 44) | (slot + 1), 0 marking an empty entry. An
// insert that finds its slot already present adds one to the count and
// learns how many equal slots were inserted before it; summed over all
// inserts that is sum_v k_v (k_v - 1) / 2 = the number of pairs (x < y)
// with slots[x] == slots[y], whatever the insertion order. The table has at
// least twice as many entries as slots, so every probe sequence ends.
//
// Fused decode + KV write precondition (mv_paged_decode_write).
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
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "mv_common.h"

namespace mv {

// The step check's arguments (mv_decode_step_check): the slot check of the
// step's decode slots, phase 1 of the fused-write check, the positions
// check and the gather of the rotary tables' rows at each position.
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

// Validates mv_decode_step_check's arguments (`who` names the entry point
// in the messages) and fills `a`; the writers' table goes to `workspace`.
int step_check_prepare(const char* who, const int64_t* slot_mapping, const void* block_table,
                       int64_t bt_stride, const void* kv_len, int32_t num_seqs, int32_t max_blocks,
                       int32_t block_size, int64_t num_blocks, const int64_t* positions,
                       const void* cos_table, const void* sin_table, int64_t table_stride,
                       int64_t max_positions, int32_t head_dim, int32_t dtype, void* cos_rows,
                       void* sin_rows, int32_t* status, void* workspace, size_t workspace_bytes,
                       StepCheckArgs* a);

// Enqueues phase 2 of the fused-write check (the shared-read scan) after a
// step check with arguments `a` has run on the stream.
int step_check_scan(const StepCheckArgs& a, int32_t bt_is_i64, int32_t kv_len_is_i64, hipStream_t s);

// Enqueues the step check (one work group) and its shared-read scan.
int step_check_launch(const StepCheckArgs& a, int32_t bt_is_i64, int32_t kv_len_is_i64, hipStream_t s);

inline uint32_t pow2_at_least(int64_t v) {
  uint32_t h = 1;
  while (h < v) h <<= 1;
  return h;
}

namespace {

constexpr int kSlotCountShift = 44;
constexpr uint64_t kSlotKeyMask = (uint64_t(1) << kSlotCountShift) - 1;

constexpr int kWriteCheckThreads = 1024;
constexpr int kWriteCheckEntries = 2 * MV_WRITE_CHECK_MAX_SEQS;  // 64 KiB of LDS
constexpr int kWriterSeqBits = 12;  // MV_WRITE_CHECK_MAX_SEQS = 1 << 12
constexpr int kWriterMaxBlockLog2 = 20;  // offsets < 2^20 fit the value's upper bits
static_assert(kWriterMaxBlockLog2 + kWriterSeqBits <= 32, "writer value bits");
constexpr int kSharedCheckThreads = 256;
static_assert(MV_WRITE_CHECK_MAX_SEQS == (1 << kWriterSeqBits), "writer index bits");

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

__device__ __forceinline__ uint32_t hash32(uint32_t k) { return (k * 0x9E3779B1u) >> 7; }

// Phase 1 for one work group of THREADS threads and at most MAXS
// sequences (called by every thread): builds the writers' table in `table`
// (LDS, hmask + 1 entries) and stores it to `writers`; returns, in every
// thread, the own-slot failures and the blocks whose smallest written
// offset has two or more writers. `dup_blocks` (LDS, (hmask + 1) / 32
// words) and `s_red` (LDS, 2 ints) are scratch.
template <int THREADS, int MAXS, typename KV, typename BT>
__device__ __forceinline__ int2 build_writers(const int64_t* slots, const BT* bt, int64_t bt_stride,
                                              const KV* kv_len, int32_t num_seqs, int32_t max_blocks,
                                              int32_t bs_log2, uint64_t* writers, uint32_t hmask,
                                              uint64_t* table, uint32_t* dup_blocks, int* s_red) {
  constexpr int kMine = (MAXS + THREADS - 1) / THREADS;
  const uint32_t dup_words = (hmask + 1 + 31) / 32;
  for (uint32_t i = threadIdx.x; i <= hmask; i += THREADS) table[i] = 0;
  for (uint32_t i = threadIdx.x; i < dup_words; i += THREADS) dup_blocks[i] = 0;
  if (threadIdx.x == 0) { s_red[0] = 0; s_red[1] = 0; }
  __syncthreads();
  int bad = 0;
  uint64_t mine[kMine];  // this thread's writers' words (0: none)
#pragma unroll
  for (int i = 0; i < kMine; ++i) mine[i] = 0;
#pragma unroll
  for (int i = 0; i < kMine; ++i) {
    const int b = static_cast<int>(threadIdx.x) + i * THREADS;
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
  for (uint32_t i = threadIdx.x; i < dup_words; i += THREADS) dups += __popc(dup_blocks[i]);
  if (dups) atomicAdd(&s_red[1], dups);
  for (uint32_t i = threadIdx.x; i <= hmask; i += THREADS) writers[i] = table[i];
  __syncthreads();
  return make_int2(s_red[0], s_red[1]);
}

// The step check in one work group of THREADS threads, at most MAXS
// sequences (called by every thread): the rotary rows, the slot check in
// `slot_table` (LDS, slot_hmask + 1 entries), phase 1 in `table` and
// `dup_blocks` (as build_writers), then the status words. `s_red`,
// `s_cnt` (2 ints each) and `s_pairs` are LDS scratch.
template <typename KV, typename BT, int THREADS, int MAXS>
__device__ __forceinline__ void step_check_body(const StepCheckArgs& a, uint64_t* slot_table, uint64_t* table,
                                                uint32_t* dup_blocks, int* s_red, int* s_cnt,
                                                unsigned long long* s_pairs) {
  for (uint32_t i = threadIdx.x; i <= a.slot_hmask; i += THREADS) slot_table[i] = 0;
  if (threadIdx.x == 0) { s_cnt[0] = 0; s_cnt[1] = 0; *s_pairs = 0; }
  // rotary rows: chunk i of 16 bytes of row b of table tb (the loads of
  // every chunk go out before any other work waits on memory)
  int pos_bad = 0;
  if (a.positions) {
    const int cpr = a.row_bytes / 16;
    const int n = 2 * a.num_seqs * cpr;
    for (int i = threadIdx.x; i < n; i += THREADS) {
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
  for (int x = threadIdx.x; x < a.num_seqs; x += THREADS) {
    const int64_t s = a.slots[x];
    if (s == -1) continue;
    if (s < 0 || s >= a.total_slots) { ++bad; continue; }
    pairs += count_insert(slot_table, a.slot_hmask, static_cast<uint64_t>(s) + 1);
  }
  if (bad) atomicAdd(&s_cnt[0], bad);
  if (pairs) atomicAdd(s_pairs, static_cast<unsigned long long>(pairs));
  if (pos_bad) atomicAdd(&s_cnt[1], pos_bad);
  const int2 r = build_writers<THREADS, MAXS>(a.slots, static_cast<const BT*>(a.bt), a.bt_stride,
                                              static_cast<const KV*>(a.kv_len), a.num_seqs, a.max_blocks,
                                              a.bs_log2, a.writers, a.writer_hmask, table, dup_blocks, s_red);
  if (threadIdx.x == 0) {  // build_writers ends on a barrier: the counts are complete
    a.status[MV_STEP_SLOTS_OUT_OF_RANGE] = s_cnt[0];
    a.status[MV_STEP_SLOTS_DUPLICATES] = saturate_i32(*s_pairs);
    a.status[MV_STEP_WRITE_OWN_SLOT] = r.x;
    a.status[MV_STEP_WRITE_SHARED] = r.y;
    a.status[MV_STEP_POSITIONS] = s_cnt[1];
  }
}

}  // namespace
}  // namespace mv
