// Shared device helpers for the gfx950 Sage attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sage {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kQK_INT8 = 0, kQK_FP8 = 1;
constexpr int kPV_BF16 = 0, kPV_FP8 = 1;
constexpr int kGRAN_TOKEN = 0, kGRAN_BLOCK64 = 1;

constexpr int kRowsPerWG = 128;  // query rows per workgroup = reference Q tile (block_mask.py:27)
constexpr int kKVTile = 64;      // keys per tile = reference KV tile (block_mask.py:28)
constexpr float kEps = 1e-12f;   // tl.maximum(amax, 1e-12) (sage_kernels.py:1421)
constexpr float kFp8Max = 448.0f;
constexpr float kInt8Max = 127.0f;

__host__ __device__ inline int64_t padded_len(int64_t n) { return (n + 127) / 128 * 128; }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// fp32 -> bf16, round to nearest even (the rounding torch uses for bf16
// results): gfx950's v_cvt_pk_bf16_f32.  NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two fp32 -> two OCP e4m3fn codes (RNE, saturating) packed into 16 bits.
__device__ __forceinline__ uint32_t pack_fp8x2(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  // the "old" operand only supplies the high half, which the second convert
  // overwrites: passing a's bits lets the result share a's register instead
  // of a zeroed one
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// Truncating fp32 -> int8 (Triton .to(tl.int8) lowers to fptosi), packed.
__device__ __forceinline__ uint32_t pack_i8x4(float a, float b, float c, float d) {
  uint32_t x0 = (uint32_t)((int)a) & 0xffu;
  uint32_t x1 = (uint32_t)((int)b) & 0xffu;
  uint32_t x2 = (uint32_t)((int)c) & 0xffu;
  uint32_t x3 = (uint32_t)((int)d) & 0xffu;
  return x0 | (x1 << 8) | (x2 << 16) | (x3 << 24);
}

// Tile class for a block of queries against one key tile:
// 0 = nothing visible, 1 = everything visible, 2 = per-token mask needed.
// Summaries are (min doc, max doc, #valid tokens, #padding tokens) over
// tokens below N (an empty one is (INT_MAX, -INT_MAX, 0, 0)); padded queries
// (doc < 0) see every valid key.
__device__ __forceinline__ int classify(int4 qsum, int4 ksum) {
  if (qsum.z + qsum.w == 0) return 0;           // no query row below N
  if (ksum.z == 0) return 0;                    // no valid key
  if (qsum.z == 0) return ksum.w == 0 ? 1 : 2;  // only padded queries: they see every valid key
  if (qsum.w == 0 && (qsum.y < ksum.x || ksum.y < qsum.x)) return 0;
  if (ksum.w == 0 && ksum.x == ksum.y && qsum.x == qsum.y && qsum.x == ksum.x) return 1;
  return 2;
}

// Summary of the union of two token blocks.
__device__ __forceinline__ int4 merge_summary(int4 a, int4 b) {
  return make_int4(min(a.x, b.x), max(a.y, b.y), a.z + b.z, a.w + b.w);
}

// Copies a region of C 16-byte chunks into LDS with direct global -> LDS
// loads (global_load_lds_dwordx4) by a workgroup of WAVES waves: wave w moves
// the 64-chunk blocks w, w + WAVES, ...; lane l of block j lands at LDS chunk
// 64 j + l, and src(x) is the global address of chunk x.  No registers hold
// the data on its way; the caller waits for vmcnt(0) (wait_vmem) before the
// barrier that publishes the stage.
template <int C, int WAVES, typename Src>
__device__ __forceinline__ void dma_chunks(uint8_t* lds, int wave, int lane, Src src) {
  static_assert(C % 64 == 0, "whole 64-chunk blocks");
#pragma unroll
  for (int j0 = 0; j0 < C / 64; j0 += WAVES) {
    const int j = j0 + wave;
    if (C / 64 % WAVES == 0 || j < C / 64)
      __builtin_amdgcn_global_load_lds(src(j * 64 + lane), lds + j * 1024, 16, 0, 0);
  }
}

// dma_chunks through a buffer resource: chunk x of the region that starts
// at byte `soff` of resource `rs` lands at LDS chunk x (the same split over
// waves).  The lane part of the offset is loop-invariant; the region and
// block parts are scalar, so no vector register holds an address.  Loads
// past the resource's size return zeros.
template <int C, int WAVES>
__device__ __forceinline__ void dma_chunks_buf(uint8_t* lds, int wave, int lane, __amdgpu_buffer_rsrc_t rs,
                                               int soff) {
  static_assert(C % 64 == 0, "whole 64-chunk blocks");
#pragma unroll
  for (int j0 = 0; j0 < C / 64; j0 += WAVES) {
    const int j = j0 + wave;
    if (C / 64 % WAVES == 0 || j < C / 64)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds + j * 1024, 16, (wave * 64 + lane) * 16, soff + j0 * 1024,
                                               0, 0);
  }
}

// Loads at a workgroup-uniform index through the constant address space, so
// the compiler emits scalar loads: they wait on the scalar counter, not behind
// direct global -> LDS loads in flight (which a vector load's vmcnt wait would
// include).
__device__ __forceinline__ int4 load_uniform(const int4* base, int64_t i) {
  typedef const __attribute__((address_space(4))) int* ConstPtr;
  const ConstPtr q = (ConstPtr)(base + i);
  return make_int4(q[0], q[1], q[2], q[3]);
}
__device__ __forceinline__ int32_t load_uniform(const int32_t* base, int64_t i) {
  typedef const __attribute__((address_space(4))) int32_t* ConstPtr;
  return *(ConstPtr)(base + i);
}
__device__ __forceinline__ float load_uniform(const float* base, int64_t i) {
  typedef const __attribute__((address_space(4))) float* ConstPtr;
  return *(ConstPtr)(base + i);
}
// Byte i of a uniform byte array, from the aligned dword that holds it.
__device__ __forceinline__ uint32_t load_uniform_u8(const uint8_t* base, int64_t i) {
  typedef const __attribute__((address_space(4))) uint32_t* ConstPtr;
  const uintptr_t a = reinterpret_cast<uintptr_t>(base + i);
  const uint32_t w = *(ConstPtr)(a & ~(uintptr_t)3);
  return (w >> (8 * (a & 3))) & 0xffu;
}

// Raw (untyped) buffer resource over `bytes` bytes at `base`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// Counts a piece's arrival at its split item's counter (tag << 8 | pieces
// arrived, relaxed agent-scope atomics); true for the last of `parts` pieces.
// A counter whose tag is not this launch's (another call's, or memory never
// written) starts again from 0.
__device__ __forceinline__ bool arrive_last(uint64_t* ctr, uint64_t tag, int parts) {
  const uint64_t mine = tag << 8;
  uint64_t old = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint64_t next;
  do {
    next = ((old & ~(uint64_t)0xff) == mine ? old : mine) + 1;
  } while (!__hip_atomic_compare_exchange_weak(ctr, &old, next, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT));
  return (int)(next & 0xff) == parts;
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left free; gfx9 encoding).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// Byte offset of the 16-byte piece of row-fragment code storage that holds
// token `tok`, channels [32*c + 16*h, +16).  See include/sage_mi355x.h.
__host__ __device__ __forceinline__ int64_t row_frag_offset(int64_t tok, int c, int h, int d) {
  const int64_t rb = tok >> 5;
  const int r = (int)(tok & 31);
  return ((rb * (d / 32) + c) * 64 + (h * 32 + r)) * 16;
}

}  // namespace sage
