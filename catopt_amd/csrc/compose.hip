// Level-batched composition of affine maps held in slot arrays (fp32).
//
// A forest of compose terms (any bracketing, shared subterms once) is
// evaluated level by level.  The leaf maps occupy slots 0 .. n-1, and the
// nodes of each level take the next consecutive slots, so one launch per
// level writes
//     slot[out0 + j] = compose(slot[f[j]], slot[g[j]]),     j < L,
// where every operand slot lies below out0 (written by an earlier launch or
// a leaf).  compose(f, g) applies g first:
//   diagonal:  (fa * ga,  fa * gb + fb)       elementwise over S lanes
//   dense:     (fa @ ga,  fa @ gb + fb)       d x d maps, P per slot
// An operand index outside [0, out0) yields NaN in that output slot (the
// host builds the index lists from the plan; this only keeps a bad list
// from reading outside the slots).
//
// The diagonal form rounds the product and the sum separately (contraction
// into a fused multiply-add is switched off), so every element equals the
// serial evaluation of the same compose term element by element.
#include "common.hpp"

namespace catopt {
namespace {

constexpr int kThreads = 256;

inline uint32_t grid_for(int64_t n) {
  int64_t g = (n + kThreads - 1) / kThreads;
  if (g > 65536) g = 65536;
  return (uint32_t)(g < 1 ? 1 : g);
}

__device__ __forceinline__ bool slot_ok(int64_t i, int64_t out0) { return i >= 0 && i < out0; }

__global__ __launch_bounds__(kThreads) void affd_compose_slots_kernel(
    int64_t S, float* __restrict__ A, float* __restrict__ B, const int64_t* __restrict__ f,
    const int64_t* __restrict__ g, int64_t L, int64_t out0) {
#pragma clang fp contract(off)
  const int64_t n = L * S;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const int64_t j = i / S, s = i - j * S;
    const int64_t fi = f[j], gi = g[j];
    float oa, ob;
    if (slot_ok(fi, out0) && slot_ok(gi, out0)) {
      const float fa = A[fi * S + s], fb = B[fi * S + s];
      const float ga = A[gi * S + s], gb = B[gi * S + s];
      oa = fa * ga;
      const float p = fa * gb;
      ob = p + fb;
    } else {
      oa = ob = __builtin_nanf("");
    }
    A[(out0 + j) * S + s] = oa;
    B[(out0 + j) * S + s] = ob;
  }
}

// One workgroup per (node, batch entry): the d x d product and the offset.
__global__ __launch_bounds__(kThreads) void aff_compose_slots_kernel(
    int64_t P, int64_t d, float* __restrict__ A, float* __restrict__ B, const int64_t* __restrict__ f,
    const int64_t* __restrict__ g, int64_t L, int64_t out0) {
  const int64_t dd = d * d;
  for (int64_t w = blockIdx.x; w < L * P; w += gridDim.x) {
    const int64_t j = w / P, p = w - j * P;
    const int64_t fi = f[j], gi = g[j];
    const bool ok = slot_ok(fi, out0) && slot_ok(gi, out0);
    float* __restrict__ oA = A + ((out0 + j) * P + p) * dd;
    float* __restrict__ oB = B + ((out0 + j) * P + p) * d;
    const float* fA = A + ((ok ? fi : 0) * P + p) * dd;
    const float* gA = A + ((ok ? gi : 0) * P + p) * dd;
    const float* fB = B + ((ok ? fi : 0) * P + p) * d;
    const float* gB = B + ((ok ? gi : 0) * P + p) * d;
    for (int64_t e = threadIdx.x; e < dd; e += kThreads) {
      const int64_t r = e / d, c = e - r * d;
      float acc = 0.f;
      for (int64_t k = 0; k < d; ++k) acc = fmaf(fA[r * d + k], gA[k * d + c], acc);
      oA[e] = ok ? acc : __builtin_nanf("");
    }
    for (int64_t r = threadIdx.x; r < d; r += kThreads) {
      float acc = 0.f;
      for (int64_t k = 0; k < d; ++k) acc = fmaf(fA[r * d + k], gB[k], acc);
      oB[r] = ok ? acc + fB[r] : __builtin_nanf("");
    }
    // the next (node, batch entry) of this workgroup writes other slots only
  }
}

int32_t check_slots(int64_t n_slots, int64_t width, const float* A, const float* B, const int64_t* f,
                    const int64_t* g, int64_t L, int64_t out0) {
  if (n_slots <= 0 || width <= 0 || L < 0 || out0 < 1 || out0 > n_slots || L > n_slots - out0)
    return CATOPT_E_INVAL;
  if (width > (int64_t(1) << 40) / n_slots) return CATOPT_E_UNSUPPORTED;
  if (L > 0 && (!A || !B || !f || !g)) return CATOPT_E_INVAL;
  return CATOPT_OK;
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int32_t catopt_hip_affd_compose_slots(int64_t n_slots, int64_t S, float* A, float* B,
                                                 const int64_t* f, const int64_t* g, int64_t L,
                                                 int64_t out0, void* stream) {
  const int32_t st = check_slots(n_slots, S, A, B, f, g, L, out0);
  if (st != CATOPT_OK || L == 0) return st;
  affd_compose_slots_kernel<<<grid_for(L * S), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      S, A, B, f, g, L, out0);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

extern "C" int32_t catopt_hip_aff_compose_slots(int64_t n_slots, int64_t P, int64_t d, float* A,
                                                float* B, const int64_t* f, const int64_t* g, int64_t L,
                                                int64_t out0, void* stream) {
  if (P <= 0 || d <= 0 || d > 4096) return CATOPT_E_INVAL;
  const int32_t st = check_slots(n_slots, P * d * d, A, B, f, g, L, out0);
  if (st != CATOPT_OK || L == 0) return st;
  const int64_t blocks = L * P < 65536 ? L * P : 65536;
  aff_compose_slots_kernel<<<dim3((uint32_t)blocks), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      P, d, A, B, f, g, L, out0);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}
