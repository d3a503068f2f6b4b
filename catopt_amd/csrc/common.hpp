// Shared device/host helpers for the gfx950 kernels of libcatopt_hip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "catopt_hip.h"

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

namespace catopt {

// Record a failed HIP call for catopt_hip_last_hip_error(); returns CATOPT_E_HIP.
int32_t set_hip_error(hipError_t e);

#define CATOPT_LAUNCH_CHECK()                                   \
  do {                                                          \
    hipError_t e_ = hipGetLastError();                          \
    if (e_ != hipSuccess) return ::catopt::set_hip_error(e_);   \
  } while (0)

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}

// Two fp32 -> one dword of bf16 (lo in bits 0..15), round-to-nearest-even;
// written as a 2-vector conversion so it lowers to one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p, int64_t i);
template <>
__device__ __forceinline__ float load_f32<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float load_f32<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_to_f32(p[i]);
}

template <typename T>
__device__ __forceinline__ void store_f32(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void store_f32<float>(float* p, int64_t i, float v) {
  p[i] = v;
}
template <>
__device__ __forceinline__ void store_f32<uint16_t>(uint16_t* p, int64_t i, float v) {
  p[i] = f32_to_bf16(v);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }
__device__ __forceinline__ float sigmoid_f(float g) { return 1.0f / (1.0f + __expf(-g)); }

// 32x32x16 bf16 MFMA (gfx950).  Operand lane layout: lane l supplies row
// (l % 32) of A and column (l % 32) of B, each with 8 consecutive k values of
// its half-wave group (l / 32).  Accumulator: lane l holds column (l % 32),
// rows 8*(r/4) + 4*(l/32) + (r%4) for r = 0..15.
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row of accumulator register r for half-wave group g (0/1).
__device__ __forceinline__ constexpr int acc_row(int r, int g) {
  return 8 * (r >> 2) + 4 * g + (r & 3);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// γ^k for an integer k >= 0 from lg = log2|γ| and neg = (γ < 0), as pow
// gives it for an integer exponent: 1 at k = 0 (0^0 included, where
// exp2(0 · log2 0) would be NaN) and, for a negative γ, the sign of k's
// parity.
__device__ __forceinline__ float pow_k(float lg, bool neg, int k) {
  const float r = k == 0 ? 1.f : __builtin_amdgcn_exp2f((float)k * lg);
  return (neg && (k & 1)) ? -r : r;
}

// LDS byte address of a pointer into dynamic shared memory.
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// Direct global->LDS load of 16 bytes per lane: lane l's bytes land at LDS
// byte address lds_wave + 16 l (lds_wave is wave-uniform; it goes to M0).
// Issued as inline asm: for the builtin form the compiler treats every later
// transposing LDS read (ds_read_b64_tr_b16) as a possible reader of the load
// and waits for all loads in flight before it, which serialises a prefetch
// with the tile being computed.  Callers wait with s_waitcnt vmcnt before
// the barrier that publishes the loaded stage.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_wave) {
  // one wait state between the SALU write of M0 and the LDS-DMA load that
  // reads it (a hazard the compiler cannot see inside inline asm)
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_wave)
               : "m0");
}

// Direct global->LDS load of 4 bytes per lane (lane l's word lands at
// lds_wave + 4 l), as dma16: inline asm, so the compiler neither waits for it
// before unrelated LDS accesses nor counts it; callers wait with s_waitcnt
// vmcnt before the barrier that publishes the data.
__device__ __forceinline__ void dma4(const void* gptr, uint32_t lds_wave) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(gptr), "s"(lds_wave)
               : "m0");
}

// One 1 KB global->LDS load through a buffer resource: lane l's 16 bytes at
// byte `voff` of the buffer land at LDS byte address lds + 16 l (lds is
// wave-uniform; it goes to M0).  A load past the resource's range returns
// zeros.  The s_nop is the one wait state the hardware needs between an SALU
// write of M0 and an LDS-DMA load reading it (the compiler cannot insert it
// inside inline asm; without it the load can take the previous M0 and land in
// another load's place).  Inline asm for the reason given at dma16.
// `lds` goes through readfirstlane: under SGPR pressure the compiler may hold
// a uniform value in a VGPR, which an "s" operand cannot take.
__device__ __forceinline__ void dma_buf(u32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(lds)) : "m0", "memory");
}

// Buffer resource (raw, stride 0) over `bytes` bytes from `base`.
__device__ __forceinline__ u32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  r.z = __builtin_amdgcn_readfirstlane(bytes);
  r.w = 0x00020000;
  return r;
}

}  // namespace catopt
