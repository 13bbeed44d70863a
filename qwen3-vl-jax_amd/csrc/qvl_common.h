// Shared device/host helpers for the gfx950 kernels of libqvl.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "qvl_vision.h"

namespace qvl {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Buffer resource word 3 for gfx9-family (CDNA) raw buffer accesses.
constexpr int kBufferRsrcWord3 = 0x00020000;

// Raw buffer resource over [base, base + bytes): loads past the end return zeros, which is how
// the kernels read ragged tails without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferRsrcWord3);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

__device__ __forceinline__ u32x2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even float -> bf16 pair packed in one dword (lo = a, hi = b).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// Value of `x` after rounding to bf16 (kept as float).
__device__ __forceinline__ float round_bf16(float x) { return (float)(__bf16)x; }

__device__ __forceinline__ float gelu_tanh(float x) {
  // jax.nn.gelu(approximate=True): 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3).
  // Identity 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)), and -2u log2(e) = x (c0 + c1 x^2) with
  // c0 = -2 log2(e) sqrt(2/pi), c1 = 0.044715 c0; exp via the hardware exp2. Saturates
  // correctly: exp2 -> inf gives (-)0, exp2 -> 0 gives x.
  const float c0 = -2.3022082f;                 // -2 * log2(e) * sqrt(2/pi)
  const float c1 = -0.10294324f;                // 0.044715 * c0
  const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(c1, x * x, c0));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// Raw buffer resource words (base, stride 0, byte range, gfx9 word 3) for the asm DMA below.
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, (uint32_t)kBufferRsrcWord3};
}

// 16 bytes per lane, global -> LDS: lane i writes LDS bytes [M0 + 16 i, M0 + 16 i + 16), M0 = lds.
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(soff), "s"(lds) : "memory", "m0");
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__host__ __device__ constexpr int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// XCD-aware remap of a linear workgroup id: the dispatcher deals workgroups round-robin over the
// 8 XCDs (wg % 8); this returns a tile id such that each XCD walks a contiguous range of tiles,
// so tiles sharing operands also share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int wg, int n) {
  const int q = n >> 3, r = n & 7;
  const int xcd = wg & 7, idx = wg >> 3;
  return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

}  // namespace qvl

// Error plumbing shared by the host entry points (set_error in qvl_meta.cpp, check_launch in
// qvl_host.hip).
namespace qvl {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
}  // namespace qvl
