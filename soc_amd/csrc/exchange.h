// exchange.h - tagged 32-bit words for hand-offs between the blocks of a persistent kernel (gfx950).
//
// A word holds an fp32 value rounded to nearest at 21 mantissa bits with a 2-bit phase tag in its two low bits.
// Readers spin until the words they need carry the expected tag. An aligned 4-byte store is single-copy atomic, so a
// value is never seen without its tag and no barrier or cache maintenance is needed. Two tag bits suffice when every
// word is written once per phase and a producer can only reach phase p + 1 after every reader has consumed phase p.
//
// Visibility on MI355X (measured): a device-scope (sc1) store is seen by sc1 loads on every XCD; a plain store is
// seen by sc1 loads of blocks on the same XCD only (the line stays in that XCD's L2), with half the round-trip
// latency (about 450 ns vs 900 ns for a ping-pong). Loads without sc1 may hit stale L1 lines and are never used to
// poll.
#pragma once

#include "device_common.h"

namespace soc {

__device__ __forceinline__ uint64_t now_ticks() { return __builtin_amdgcn_s_memrealtime(); }

// Tagged exchange word: value rounded to nearest at 21 mantissa bits (relative error <= 2^-22), tag in bits 0..1.
__device__ __forceinline__ uint32_t tw_pack(float v, uint32_t tag) { return ((__float_as_uint(v) + 2u) & ~3u) | tag; }
__device__ __forceinline__ float tw_val(uint32_t w) { return __uint_as_float(w & ~3u); }
__device__ __forceinline__ uint32_t tw_tag(uint32_t w) { return w & 3u; }
// Four words carry tag t when every byte-0 tag field equals t (out-of-range quads are filled with t).
__device__ __forceinline__ bool tw_quad_ok(const u32x4& w, uint32_t tag) {
  return ((w.x & 3u) == tag) & ((w.y & 3u) == tag) & ((w.z & 3u) == tag) & ((w.w & 3u) == tag);
}

__device__ __forceinline__ void ll_store(uint32_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, tw_pack(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t ll_peek(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool err_raised(int* err) {
  return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Back-off between polling rounds: fewer re-reads of lines that producers are about to write.
__device__ __forceinline__ void poll_pause(int n) {
  for (int i = 0; i < n; ++i) __builtin_amdgcn_s_sleep(1);
}

// Pollers keep two reads of the same words in flight, the second issued about half a read's round trip after the
// first (s_sleep units of 64 clocks): a word that lands just after one read left is seen by the other half a round
// trip later instead of a whole one. Loads return in order, so checking the older read waits for it alone.
constexpr int kStaggerLocal = 2;   // XCD-local words (plain stores, sc1 reads)
constexpr int kStaggerRemote = 8;  // words written by other XCDs (sc1 stores)
template <int N>
__device__ __forceinline__ void stagger() {
  __builtin_amdgcn_s_sleep(N);
}

// Plain store (no cache-policy bits) of a tagged word to word `idx` of the region at `base` (block-uniform):
// visible to sc1 loads of blocks on the writer's XCD only.
__device__ __forceinline__ void ll_store_local(uint32_t* base, int idx, float v, uint32_t tag) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b32(tw_pack(v, tag), r, idx * 4, 0, 0);
}

// Device-scope (sc1) store of a tagged word to word `idx` of the region at `base` (block-uniform): visible to sc1
// loads on every XCD. The base stays in scalar registers and the lane needs only a 32-bit offset.
__device__ __forceinline__ void ll_store_buf(uint32_t* base, int idx, float v, uint32_t tag) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b32(tw_pack(v, tag), r, idx * 4, 0, 16);
}

// Relaxed device-scope read of four tagged words through a buffer resource (sc1: coherent across XCDs). The lane's
// byte offset stays in one register and the per-chunk part folds into the instruction's offset fields, so a
// receiver polling thousands of elements needs no per-element address registers. Each aligned 4-byte word of the
// 16-byte load is single-copy atomic on its own, and each carries its own tag.
__device__ __forceinline__ u32x4 ll_peek_buf4(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16);
}

}  // namespace soc
