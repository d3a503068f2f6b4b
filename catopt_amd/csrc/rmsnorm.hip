// Fused RMSNorm: one HBM read of x, one write of y.
//
// y[r,:] = x[r,:] * rsqrt(mean(x[r,:]^2) + eps) * w
//
// Fast path (bf16/fp32, 16-byte aligned rows, cols a multiple of the vector
// width, cols <= 256 threads * VPT vectors): the whole row lives in
// registers between the reduction and the scaling, so x is read exactly
// once.  Generic path: two passes over the row (second pass hits L2).
#include "common.hpp"

namespace catopt {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) s += red[i];
  return s;
}

// bf16 rows held in registers: VPT 16-byte vectors (8 elements) per thread.
template <int VPT>
__global__ __launch_bounds__(kThreads) void rmsnorm_bf16_reg(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w,
    float eps, uint16_t* __restrict__ y, int64_t ldy, int cols) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * ldx);
  const int nvec = cols / 8;
  u32x4 v[VPT];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c < nvec) {
      v[i] = __builtin_nontemporal_load(xr + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float lo = __uint_as_float(v[i][j] << 16), hi = __uint_as_float(v[i][j] & 0xffff0000u);
        ss += lo * lo + hi * hi;
      }
    }
  }
  const float tot = block_sum(ss, red);
  const float r = rsqrtf(tot / static_cast<float>(cols) + eps);
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  u32x4* yr = reinterpret_cast<u32x4*>(y + row * ldy);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c < nvec) {
      u32x4 wv;
      if (w) wv = wr[c];
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float lo = __uint_as_float(v[i][j] << 16) * r, hi = __uint_as_float(v[i][j] & 0xffff0000u) * r;
        if (w) {
          lo *= __uint_as_float(wv[j] << 16);
          hi *= __uint_as_float(wv[j] & 0xffff0000u);
        }
        o[j] = pack_bf16x2(lo, hi);
      }
      __builtin_nontemporal_store(o, yr + c);
    }
  }
}

template <int VPT>
__global__ __launch_bounds__(kThreads) void rmsnorm_f32_reg(
    const float* __restrict__ x, int64_t ldx, const float* __restrict__ w, float eps,
    float* __restrict__ y, int64_t ldy, int cols) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const f32x4* xr = reinterpret_cast<const f32x4*>(x + row * ldx);
  const int nvec = cols / 4;
  f32x4 v[VPT];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c < nvec) {
      v[i] = xr[c];
      ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
    }
  }
  const float tot = block_sum(ss, red);
  const float r = rsqrtf(tot / static_cast<float>(cols) + eps);
  const f32x4* wr = reinterpret_cast<const f32x4*>(w);
  f32x4* yr = reinterpret_cast<f32x4*>(y + row * ldy);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c < nvec) {
      f32x4 o = v[i] * r;
      if (w) o *= wr[c];
      yr[c] = o;
    }
  }
}

// Generic two-pass path: any alignment, any cols.
template <typename T>
__global__ __launch_bounds__(kThreads) void rmsnorm_generic(
    const T* __restrict__ x, int64_t ldx, const T* __restrict__ w, float eps,
    T* __restrict__ y, int64_t ldy, int64_t cols) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ldx;
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    float f = load_f32(xr, c);
    ss += f * f;
  }
  const float tot = block_sum(ss, red);
  const float r = rsqrtf(tot / static_cast<float>(cols) + eps);
  T* yr = y + row * ldy;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    float f = load_f32(xr, c) * r;
    if (w) f *= load_f32(w, c);
    store_f32(yr, c, f);
  }
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int32_t catopt_hip_rmsnorm(int32_t dtype, int64_t rows, int64_t cols,
                                      const void* x, int64_t ldx, const void* w, float eps,
                                      void* y, int64_t ldy, void* stream) {
  if (rows < 0 || cols <= 0 || ldx < cols || ldy < cols) return CATOPT_E_INVAL;
  if (rows == 0) return CATOPT_OK;
  if (!x || !y) return CATOPT_E_INVAL;
  if (rows > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(rows)), block(kThreads);
  if (dtype == CATOPT_BF16) {
    auto xp = static_cast<const uint16_t*>(x);
    auto wp = static_cast<const uint16_t*>(w);
    auto yp = static_cast<uint16_t*>(y);
    const bool vec = cols % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && aligned16(x) &&
                     aligned16(y) && (!w || aligned16(w));
    const int64_t nvec = cols / 8;
    if (vec && nvec <= kThreads * 1)
      rmsnorm_bf16_reg<1><<<grid, block, 0, s>>>(xp, ldx, wp, eps, yp, ldy, (int)cols);
    else if (vec && nvec <= kThreads * 2)
      rmsnorm_bf16_reg<2><<<grid, block, 0, s>>>(xp, ldx, wp, eps, yp, ldy, (int)cols);
    else if (vec && nvec <= kThreads * 4)
      rmsnorm_bf16_reg<4><<<grid, block, 0, s>>>(xp, ldx, wp, eps, yp, ldy, (int)cols);
    else if (vec && nvec <= kThreads * 8)
      rmsnorm_bf16_reg<8><<<grid, block, 0, s>>>(xp, ldx, wp, eps, yp, ldy, (int)cols);
    else
      rmsnorm_generic<uint16_t><<<grid, block, 0, s>>>(xp, ldx, wp, eps, yp, ldy, cols);
  } else if (dtype == CATOPT_F32) {
    auto xp = static_cast<const float*>(x);
    auto wp = static_cast<const float*>(w);
    auto yp = static_cast<float*>(y);
    const bool vec = cols % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && aligned16(x) &&
                     aligned16(y) && (!w || aligned16(w));
    const int64_t nvec = cols / 4;
    if (vec && nvec <= kThreads * 2)
      rmsnorm_f32_reg<2><<<grid, block, 0, s>>>(xp, ldx, wp, eps, yp, ldy, (int)cols);
    else if (vec && nvec <= kThreads * 8)
      rmsnorm_f32_reg<8><<<grid, block, 0, s>>>(xp, ldx, wp, eps, yp, ldy, (int)cols);
    else
      rmsnorm_generic<float><<<grid, block, 0, s>>>(xp, ldx, wp, eps, yp, ldy, cols);
  } else {
    return CATOPT_E_UNSUPPORTED;
  }
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}
