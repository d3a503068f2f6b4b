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
// max that propagates NaN, as torch.maximum / torch.amax do (fmaxf drops it)
__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}

__global__ __launch_bounds__(kThreads) void om_compose_kernel(
    int64_t rows, int64_t dv, const float* m1, const float* l1, const float* a1,
    const float* m2, const float* l2, const float* a2, float* m, float* l, float* a) {
  const int64_t total = rows * dv;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / dv;
    const float ma = m1[r], mb = m2[r];
    const float mx = nan_max(ma, mb);
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
    const float mx = nan_max(ma, mb);
    const bool fa = __builtin_isfinite(ma), fb = __builtin_isfinite(mb);
    const float ea = fa ? __expf(ma - mx) : 0.f;
    const float eb = fb ? __expf(mb - mx) : 0.f;
    const float lv = (fa ? l1[r] * ea : 0.f) + (fb ? l2[r] * eb : 0.f);
    l[r] = lv;
    m[r] = mx;
  }
}

// Row statistics of an explicit score block (one wave per row): a pass for
// the NaN-propagating row max, a pass writing e = exp(s - m) and summing it.
// The sum reduces in a fixed xor-tree order, so results are deterministic.
template <typename T>
__global__ __launch_bounds__(kThreads) void om_rows_kernel(int64_t rows, int64_t cols,
                                                           const T* __restrict__ s, int64_t lds,
                                                           int sanitize, float* __restrict__ m,
                                                           float* __restrict__ l,
                                                           float* __restrict__ e, int64_t lde) {
  const int64_t r = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;  // whole wave
  const T* sr = s + r * lds;
  float mx = -__builtin_inff();
  int has_nan = 0;
  for (int64_t c = lane; c < cols; c += 64) {
    const float v = load_f32(sr, c);
    has_nan |= v != v;
    mx = fmaxf(mx, v);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    has_nan |= __shfl_xor(has_nan, o, 64);
  }
  if (has_nan) mx = __builtin_nanf("");
  const bool zero = sanitize && !__builtin_isfinite(mx);
  float* er = e + r * lde;
  float sum = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float x = zero ? 0.f : __expf(load_f32(sr, c) - mx);
    er[c] = x;
    sum += x;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (lane == 0) {
    m[r] = mx;
    l[r] = sum;
  }
}

// Read-only HBM stream: every 16-byte word of src is read once and folded
// into an XOR that is stored only if it equals a sentinel, so the loads stay
// live while the kernel writes (almost) nothing.  Each workgroup reads one
// contiguous range, RD_U nontemporal 4 KB loads in flight per step (a
// grid-stride walk with four loads per lane reached 6.1-6.3 TB/s on MI355X,
// this layout 6.8-7.1).
constexpr int RD_U = 8;
__global__ __launch_bounds__(kThreads) void hbm_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                            int64_t per, uint32_t* __restrict__ sink) {
  const int64_t beg = (int64_t)blockIdx.x * per;
  const int64_t end = beg + per < n16 ? beg + per : n16;
  u32x4 acc = {0u, 0u, 0u, 0u};
  int64_t j = beg + threadIdx.x;
  for (; j + (RD_U - 1) * kThreads < end; j += RD_U * kThreads) {
    u32x4 w[RD_U];
#pragma unroll
    for (int u = 0; u < RD_U; ++u) w[u] = __builtin_nontemporal_load(src + j + u * kThreads);
#pragma unroll
    for (int u = 0; u < RD_U; ++u) acc ^= w[u];
  }
  for (; j < end; j += kThreads) acc ^= __builtin_nontemporal_load(src + j);
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x9e3779b9u) sink[0] = x;
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

// The om combine of L carriers over the leading axis followed by the
// diagonal deferred-affine readout:
//   M = max_i m[i, r] (NaN-propagating), w_i = isfinite(m_i) ? exp(m_i − M) : 0,
//   out[r, c] = (Σ_i w_i num[i, r, c] · h[c] + Σ_i w_i num[i, r, d + c]) / Σ_i w_i l[i, r].
// One wave per row (rows grid-strided over the waves).  Lane i holds leaf
// i's m, l and weight (64 leaves per pass), so the row statistics are one
// load each and a wave reduction; the numerators are read with the lanes
// over the columns (contiguous row segments), each leaf's weight broadcast
// from its lane, the leaf loop unrolled so its loads are in flight together.
constexpr int kFoldWaves = kThreads / 64;

__device__ __forceinline__ float wave_nan_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = nan_max(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ __launch_bounds__(kThreads) void omd_fold_apply_kernel(
    int64_t L, int64_t rows, int64_t d, const float* __restrict__ m, const float* __restrict__ l,
    const float* __restrict__ num, int64_t ldn, int64_t num_sb, const float* __restrict__ h,
    float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  for (int64_t r = (int64_t)blockIdx.x * kFoldWaves + (threadIdx.x >> 6); r < rows;
       r += (int64_t)gridDim.x * kFoldWaves) {
    float mx = -__builtin_inff();
    for (int64_t j0 = 0; j0 < L; j0 += 64) {
      const int64_t j = j0 + lane;
      mx = nan_max(mx, j < L ? m[j * rows + r] : -__builtin_inff());
    }
    mx = wave_nan_max(mx);
    const float* nrow0 = num + r * ldn;
    for (int64_t c0 = 0; c0 < d; c0 += 64) {
      const int64_t c = c0 + lane;
      const bool on = c < d;
      float ls = 0.f, fa = 0.f, fb = 0.f;
      for (int64_t j0 = 0; j0 < L; j0 += 64) {
        const int64_t j = j0 + lane;
        // a leaf with no finite score is left out by select, not weighted
        // by 0: its l and numerators may be inf or NaN (torch.where in the
        // reference's reduce)
        const float mj = j < L ? m[j * rows + r] : -__builtin_inff();
        const bool fin = __builtin_isfinite(mj);
        const float w = fin ? __expf(mj - mx) : 0.f;
        ls += (j < L && fin) ? l[j * rows + r] * w : 0.f;
        const int n = (int)(L - j0 < 64 ? L - j0 : 64);
        const float* nblk = nrow0 + j0 * num_sb;
#pragma unroll 16
        for (int t = 0; t < n; ++t) {
          const float wt = __shfl(w, t);
          const bool ft = __shfl((int)fin, t) != 0;
          if (on && ft) {
            fa += nblk[t * num_sb + c] * wt;
            fb += nblk[t * num_sb + d + c] * wt;
          }
        }
      }
      ls = wave_sum(ls);
      if (on) out[r * d + c] = (fa * h[c] + fb) / ls;
    }
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

extern "C" int32_t catopt_hip_omd_fold_apply(int64_t L, int64_t rows, int64_t d, const float* m,
                                             const float* l, const float* num, int64_t ldn,
                                             int64_t num_sb, const float* h, float* out,
                                             void* stream) {
  if (L < 1 || rows < 0 || d < 0 || ldn < 2 * d || num_sb < (rows > 0 ? (rows - 1) * ldn + 2 * d : 0))
    return CATOPT_E_INVAL;
  if (rows == 0 || d == 0) return CATOPT_OK;
  if (!m || !l || !num || !h || !out) return CATOPT_E_INVAL;
  const int64_t blocks = (rows + kFoldWaves - 1) / kFoldWaves;
  omd_fold_apply_kernel<<<dim3((uint32_t)(blocks < 65536 ? blocks : 65536)), kThreads, 0,
                          static_cast<hipStream_t>(stream)>>>(L, rows, d, m, l, num, ldn, num_sb, h, out);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

extern "C" int32_t catopt_hip_om_rows(int32_t dtype, int64_t rows, int64_t cols, const void* s,
                                      int64_t lds, int32_t sanitize, float* m, float* l, float* e,
                                      int64_t lde, void* stream) {
  if (rows < 0 || cols < 0 || lds < cols || lde < cols) return CATOPT_E_INVAL;
  if (dtype != CATOPT_F32 && dtype != CATOPT_BF16) return CATOPT_E_UNSUPPORTED;
  if (rows == 0) return CATOPT_OK;
  if (!m || !l || (cols > 0 && (!s || !e))) return CATOPT_E_INVAL;
  constexpr int64_t kRowsPerBlock = kThreads / 64;
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == CATOPT_F32)
    om_rows_kernel<float><<<dim3((uint32_t)blocks), kThreads, 0, st>>>(
        rows, cols, static_cast<const float*>(s), lds, sanitize, m, l, e, lde);
  else
    om_rows_kernel<uint16_t><<<dim3((uint32_t)blocks), kThreads, 0, st>>>(
        rows, cols, static_cast<const uint16_t*>(s), lds, sanitize, m, l, e, lde);
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

extern "C" int32_t catopt_hip_hbm_read(const void* src, int64_t nbytes, uint32_t* sink, void* stream) {
  if (nbytes < 0 || (nbytes & 15)) return CATOPT_E_INVAL;
  if (nbytes == 0) return CATOPT_OK;
  if (!src || !sink || !aligned16(src)) return CATOPT_E_INVAL;
  const int64_t n16 = nbytes / 16;
  // 512 workgroups (two per CU), each a contiguous range of whole RD_U x 4 KB
  // steps; small buffers take fewer workgroups
  constexpr int64_t step = (int64_t)RD_U * kThreads;
  int64_t blocks = (n16 + step - 1) / step;
  if (blocks > 512) blocks = 512;
  const int64_t per = ((n16 + blocks - 1) / blocks + step - 1) / step * step;
  blocks = (n16 + per - 1) / per;
  hbm_read_kernel<<<dim3((uint32_t)blocks), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4*>(src), n16, per, sink);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}
