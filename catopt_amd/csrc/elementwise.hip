// Elementwise kernels behind the generic evaluator's bindings and the om /
// decay carrier helpers.  Grid-stride, 16-byte vectorised where aligned.
#include "common.hpp"

namespace catopt {
namespace {

constexpr int kThreads = 256;

inline uint32_t grid_for(int64_t n) {
  int64_t g = (n + kThreads - 1) / kThreads;
  if (g > 65536) g = 65536;
  return (uint32_t)(g < 1 ? 1 : g);
}

template <typename T, int OP>  // OP 0: silu(x); 1: silu(g) * u
__global__ __launch_bounds__(kThreads) void unary_kernel(const T* __restrict__ x,
                                                         const T* __restrict__ u,
                                                         T* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const float g = load_f32(x, i);
    float o = silu_f(g);
    if (OP == 1) o *= load_f32(u, i);
    store_f32(y, i, o);
  }
}

template <int OP>
int32_t unary_launch(int32_t dtype, int64_t n, const void* x, const void* u, void* y, hipStream_t s) {
  if (n < 0) return CATOPT_E_INVAL;
  if (n == 0) return CATOPT_OK;
  if (!x || !y || (OP == 1 && !u)) return CATOPT_E_INVAL;
  if (dtype == CATOPT_BF16)
    unary_kernel<uint16_t, OP><<<grid_for(n), kThreads, 0, s>>>(
        static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(u), static_cast<uint16_t*>(y), n);
  else if (dtype == CATOPT_F32)
    unary_kernel<float, OP><<<grid_for(n), kThreads, 0, s>>>(
        static_cast<const float*>(x), static_cast<const float*>(u), static_cast<float*>(y), n);
  else
    return CATOPT_E_UNSUPPORTED;
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

// om_compose over rows; a is [rows, dv].  One thread per a element; the
// m/l outputs are written by the dv == 0 thread of each row after all
// threads of the row have read m1/m2/l1/l2 (outputs may alias input 1, so
// each thread reads its scalars before any write of the same row).
__global__ __launch_bounds__(kThreads) void om_compose_kernel(
    int64_t rows, int64_t dv, const float* m1, const float* l1, const float* a1,
    const float* m2, const float* l2, const float* a2, float* m, float* l, float* a) {
  const int64_t total = rows * dv;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / dv;
    const float ma = m1[r], mb = m2[r];
    const float mx = fmaxf(ma, mb);
    const bool fa = __builtin_isfinite(ma), fb = __builtin_isfinite(mb);
    const float ea = fa ? __expf(ma - mx) : 0.f;
    const float eb = fb ? __expf(mb - mx) : 0.f;
    const float av = fa ? a1[i] * ea : 0.f;
    const float bv = fb ? a2[i] * eb : 0.f;
    a[i] = av + bv;
  }
}

__global__ __launch_bounds__(kThreads) void om_compose_ml_kernel(
    int64_t rows, const float* m1, const float* l1, const float* m2, const float* l2, float* m,
    float* l) {
  for (int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x; r < rows;
       r += (int64_t)gridDim.x * kThreads) {
    const float ma = m1[r], mb = m2[r];
    const float mx = fmaxf(ma, mb);
    const bool fa = __builtin_isfinite(ma), fb = __builtin_isfinite(mb);
    const float ea = fa ? __expf(ma - mx) : 0.f;
    const float eb = fb ? __expf(mb - mx) : 0.f;
    const float lv = (fa ? l1[r] * ea : 0.f) + (fb ? l2[r] * eb : 0.f);
    l[r] = lv;
    m[r] = mx;
  }
}

// decay(γ, t)[h, i, j] = γ_h^(i-j) (i >= j) else 0
__global__ __launch_bounds__(kThreads) void decay_kernel(int64_t H, int64_t t,
                                                         const float* __restrict__ gamma,
                                                         float* __restrict__ out) {
  const int64_t total = H * t * t;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kThreads) {
    const int64_t h = e / (t * t), ij = e % (t * t), i = ij / t, j = ij % t;
    out[e] = i >= j ? powf(gamma[h], (float)(i - j)) : 0.f;
  }
}

// decay_vec(γ, t, offset, sign)[h, k] = γ_h^(sign*k + offset)
__global__ __launch_bounds__(kThreads) void decay_vec_kernel(int64_t H, int64_t t, int64_t offset,
                                                             int64_t sign,
                                                             const float* __restrict__ gamma,
                                                             float* __restrict__ out) {
  const int64_t total = H * t;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kThreads) {
    const int64_t h = e / t, k = e % t;
    out[e] = powf(gamma[h], (float)(sign * k + offset));
  }
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int32_t catopt_hip_silu(int32_t dtype, int64_t n, const void* x, void* y, void* stream) {
  return unary_launch<0>(dtype, n, x, nullptr, y, static_cast<hipStream_t>(stream));
}

extern "C" int32_t catopt_hip_silu_mul(int32_t dtype, int64_t n, const void* g, const void* u,
                                       void* y, void* stream) {
  return unary_launch<1>(dtype, n, g, u, y, static_cast<hipStream_t>(stream));
}

extern "C" int32_t catopt_hip_om_compose(int64_t rows, int64_t dv, const float* m1,
                                         const float* l1, const float* a1, const float* m2,
                                         const float* l2, const float* a2, float* m, float* l,
                                         float* a, void* stream) {
  if (rows < 0 || dv < 0) return CATOPT_E_INVAL;
  if (rows == 0) return CATOPT_OK;
  if (!m1 || !l1 || !m2 || !l2 || !m || !l || (dv > 0 && (!a1 || !a2 || !a))) return CATOPT_E_INVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // a first (reads m1/m2), then m/l: the second launch is ordered after the
  // first on the stream, so aliasing m == m1 is safe.
  if (dv > 0) {
    om_compose_kernel<<<grid_for(rows * dv), kThreads, 0, s>>>(rows, dv, m1, l1, a1, m2, l2, a2, m, l, a);
    CATOPT_LAUNCH_CHECK();
  }
  om_compose_ml_kernel<<<grid_for(rows), kThreads, 0, s>>>(rows, m1, l1, m2, l2, m, l);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

extern "C" int32_t catopt_hip_decay(int64_t H, int64_t t, const float* gamma, float* out,
                                    void* stream) {
  if (H < 0 || t < 0) return CATOPT_E_INVAL;
  if (H == 0 || t == 0) return CATOPT_OK;
  if (!gamma || !out) return CATOPT_E_INVAL;
  decay_kernel<<<grid_for(H * t * t), kThreads, 0, static_cast<hipStream_t>(stream)>>>(H, t, gamma, out);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

extern "C" int32_t catopt_hip_decay_vec(int64_t H, int64_t t, int64_t offset, int64_t sign,
                                        const float* gamma, float* out, void* stream) {
  if (H < 0 || t < 0) return CATOPT_E_INVAL;
  if (H == 0 || t == 0) return CATOPT_OK;
  if (!gamma || !out) return CATOPT_E_INVAL;
  decay_vec_kernel<<<grid_for(H * t), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      H, t, offset, sign, gamma, out);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}
