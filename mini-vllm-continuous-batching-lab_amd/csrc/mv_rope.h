// Rotary position embedding arithmetic shared by the RoPE + KV-write kernel
// and the decode kernel's fused RoPE (gfx950).
//
// The reference rotates with eager PyTorch ops in the tensors' dtype
// (RotaryEmbedding.__call__ / _rotate_half, mini_vllm/model/rotary.py:44-82):
//   x * cos + rotate_half(x) * sin,  rotate_half(x) = [-x2, x1],
// three rounded operations per element, t1 = fl(x * c), t2 = fl(r * s),
// out = fl(t1 + t2), each evaluated in fp32 and rounded to the storage type
// (what torch does for bf16 / fp16 elementwise ops; for fp32 they are
// single IEEE operations, with no fused multiply-add). With these helpers
// the outputs are bit-identical to the reference's.
#pragma once

#include "mv_common.h"

namespace mv {
namespace {

// 16 bytes of elements of one type, moved as one uint4.
template <typename T> struct Chunk16 { T e[16 / sizeof(T)]; };

template <int DTYPE>
__device__ __forceinline__ Chunk16<typename Elem<DTYPE>::raw> load16(const char* p) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  return __builtin_bit_cast(Chunk16<typename Elem<DTYPE>::raw>, v);
}

template <int DTYPE>
__device__ __forceinline__ void store16(char* p, const Chunk16<typename Elem<DTYPE>::raw>& c) {
  *reinterpret_cast<uint4*>(p) = __builtin_bit_cast(uint4, c);
}

// fl(fl(a * b) +/- fl(c * d)) in the storage type, without contraction.
// The first half's term fl(fl(x1 c) + fl(-x2 s)) is taken as
// fl(fl(x1 c) - fl(x2 s)): round-to-nearest-even is symmetric, so
// fl(-x2 s) = -fl(x2 s), and t1 + (-t2) is t1 - t2 exactly.
template <int DTYPE, bool SUB>
__device__ __forceinline__ typename Elem<DTYPE>::raw rot_term(float a, float b, float c, float d) {
#pragma clang fp contract(off)
  const float t1 = to_f32<DTYPE>(from_f32<DTYPE>(a * b));
  const float t2 = to_f32<DTYPE>(from_f32<DTYPE>(c * d));
  return from_f32<DTYPE>(SUB ? t1 - t2 : t1 + t2);
}

// One 16-byte chunk of a rotated row: `own` holds the chunk's elements,
// `partner` the elements at the same offset in the other half of the row,
// `c` / `s` the cos / sin table entries at the chunk's own dims. A chunk of
// the first half (dims < D/2) gives x1 c - x2 s, of the second x2 c + x1 s.
template <int DTYPE>
__device__ __forceinline__ uint4 rotate_chunk(uint4 own, uint4 partner, uint4 c, uint4 s,
                                              bool first_half) {
  using raw = typename Elem<DTYPE>::raw;
  constexpr int E = 16 / sizeof(raw);
  const auto x = __builtin_bit_cast(Chunk16<raw>, own);
  const auto y = __builtin_bit_cast(Chunk16<raw>, partner);
  const auto cc = __builtin_bit_cast(Chunk16<raw>, c);
  const auto ss = __builtin_bit_cast(Chunk16<raw>, s);
  Chunk16<raw> out;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float u = to_f32<DTYPE>(x.e[e]), w = to_f32<DTYPE>(y.e[e]);
    const float ce = to_f32<DTYPE>(cc.e[e]), se = to_f32<DTYPE>(ss.e[e]);
    out.e[e] = first_half ? rot_term<DTYPE, true>(u, ce, w, se) : rot_term<DTYPE, false>(u, ce, w, se);
  }
  return __builtin_bit_cast(uint4, out);
}

}  // namespace
}  // namespace mv
