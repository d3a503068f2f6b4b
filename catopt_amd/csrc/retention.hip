// Chunked decayed retention (RetNet) for gfx950, bf16 in / fp32 state.
//
//   o[t] = scale * sum_{s <= t} γ^(t-s) (q[t]·k[s]) v[s]
//
// computed chunk-wise with chunk length C = 64 and head dim 128, exactly the
// K-way block decomposition (diagonal blocks with decay(γ, C), strict-lower
// blocks with the rank-1 decay_vec factors γ^(r+(i-j)C) and γ^(-c)), with the
// strict-lower blocks of row i folded into the state
//   S_i = sum_{j<i} sum_c γ^((i-j)C - c) k_jc ⊗ v_jc,
//   S_{i+1} = γ^C S_i + sum_c γ^(C-c) k_ic ⊗ v_ic,
// so that chunk i's output is
//   oᵀ_i = scale * ( vᵀ_i (s_iᵀ ⊙ Dᵀ) + diag(γ^r) Sᵀ_i q_iᵀ ).
//
// Parallel schedule over (b·h) x segments of G chunks (three launches):
//   seg_state : each segment accumulates its local end state from zero;
//   seg_carry : per state element, exclusive fold over segments
//               (Start_{s+1} = γ^(C·G) Start_s + E_s), in place;
//   seg_out   : each segment re-walks its chunks from Start_s, emitting o.
// HBM traffic: k, v twice, q once, o once, plus the fp32 segment states.
//
// MFMA mapping (32x32x16 bf16, fp32 accumulate), 4 waves per workgroup:
//   wave w: query block qb = w & 1 (32 queries), value half dh = w >> 1;
//   sᵀ = k qᵀ          A = k rows (LDS), B = q fragments (registers)
//   intraᵀ = vᵀ Pᵀ     A = vᵀ (LDS, key-permuted 8-byte runs), B = Pᵀ from
//                      the sᵀ accumulator (the attention-kernel trick)
//   crossᵀ = Sᵀ qᵀ     A = Sᵀ bf16 copy (LDS), B = q fragments
//   S += k̃ᵀ v          A = k̃ᵀ (LDS), B = vᵀ (LDS); wave w owns dk rows 32w..
#include "common.hpp"

namespace catopt {
namespace {

constexpr int NT = 256;
constexpr int CH = 64;    // chunk length
constexpr int HD = 128;   // head dim (dk = dv)
constexpr int KCH = HD / 8;

// LDS layout (bf16 elements)
constexpr int OFF_K = 0;                    // k  [64][128]  row-major, chunk-swizzled
constexpr int OFF_KT = OFF_K + CH * HD;     // k̃ᵀ [128][64] unit-swizzled
constexpr int OFF_VT = OFF_KT + HD * CH;    // vᵀ [128][64] unit-swizzled
constexpr int OFF_ST = OFF_VT + HD * CH;    // Sᵀ [128][128] bf16, chunk-swizzled
constexpr int LDS_ELEMS = OFF_ST + HD * HD;
constexpr int LDS_BYTES = LDS_ELEMS * 2;

__device__ __forceinline__ int k_off(int key, int chunk) {
  return key * HD + ((chunk ^ (key & (KCH - 1))) << 3);
}
__device__ __forceinline__ int t_off(int d, int unit) {  // [128][64] transposed tiles
  return d * CH + ((unit ^ ((d >> 1) & 15)) << 2);
}
__device__ __forceinline__ int st_off(int dv, int chunk) {
  return dv * HD + ((chunk ^ (dv & (KCH - 1))) << 3);
}

__device__ __forceinline__ bf16x8 read_t16(const uint16_t* base, int d, int unit0) {
  const u32x2 lo = *reinterpret_cast<const u32x2*>(base + t_off(d, unit0));
  const u32x2 hi = *reinterpret_cast<const u32x2*>(base + t_off(d, unit0 + 1));
  return __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
}

struct ChunkRegs {
  u32x4 k[4];  // keys 4*kk + e, d-chunk c
  u32x4 v[4];
};

__device__ __forceinline__ void load_kv(ChunkRegs& r, const uint16_t* __restrict__ k,
                                        const uint16_t* __restrict__ v, int64_t t0, int tid) {
  const int c = tid % KCH, kk = tid / KCH;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t row = t0 + 4 * kk + e;
    r.k[e] = *reinterpret_cast<const u32x4*>(k + row * HD + c * 8);
    r.v[e] = *reinterpret_cast<const u32x4*>(v + row * HD + c * 8);
  }
}

__device__ __forceinline__ uint32_t scale_bf16x2(uint32_t w, float slo, float shi) {
  return pack_bf16x2(__uint_as_float(w << 16) * slo, __uint_as_float(w & 0xffff0000u) * shi);
}

// Store k (row-major), k̃ᵀ = (γ^(C-key) k)ᵀ and vᵀ into LDS.
template <bool WITH_K>
__device__ __forceinline__ void store_kv(uint16_t* lds, const ChunkRegs& r, float lg, int tid) {
  const int c = tid % KCH, kk = tid / KCH;
  if (WITH_K) {
#pragma unroll
    for (int e = 0; e < 4; ++e) *reinterpret_cast<u32x4*>(lds + OFF_K + k_off(4 * kk + e, c)) = r.k[e];
  }
  float kd[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) kd[e] = __builtin_amdgcn_exp2f((float)(CH - (4 * kk + e)) * lg);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int sh = (e & 1) * 16, w = e >> 1;
    uint32_t kv[4], vv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t kb = (r.k[j][w] >> sh) & 0xffffu;
      kv[j] = f32_to_bf16(__uint_as_float(kb << 16) * kd[j]);
      vv[j] = (r.v[j][w] >> sh) & 0xffffu;
    }
    const int d = c * 8 + e;
    *reinterpret_cast<u32x2*>(lds + OFF_KT + t_off(d, kk)) = u32x2{kv[0] | (kv[1] << 16), kv[2] | (kv[3] << 16)};
    *reinterpret_cast<u32x2*>(lds + OFF_VT + t_off(d, kk)) = u32x2{vv[0] | (vv[1] << 16), vv[2] | (vv[3] << 16)};
  }
}

// S[dk = 32*w + row][dv = 32*cb + l32] accumulators: S = γ^C S + k̃ᵀ v.
__device__ __forceinline__ void state_update(f32x16 (&S)[4], const uint16_t* lds, float gC,
                                             int wave, int l32, int g) {
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) S[cb][r] *= gC;
#pragma unroll
  for (int j = 0; j < CH / 16; ++j) {
    const bf16x8 a = read_t16(lds + OFF_KT, 32 * wave + l32, 4 * j + 2 * g);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const bf16x8 b = read_t16(lds + OFF_VT, 32 * cb + l32, 4 * j + 2 * g);
      S[cb] = mfma32x32x16(a, b, S[cb]);
    }
  }
}

struct SegGeom {
  int64_t bh, seg, c0, c1;  // chunk range [c0, c1)
};

__device__ __forceinline__ SegGeom seg_geom(int nseg, int G, int64_t nchunks) {
  SegGeom s;
  s.bh = blockIdx.x / nseg;
  s.seg = blockIdx.x % nseg;
  s.c0 = s.seg * G;
  s.c1 = s.c0 + G < nchunks ? s.c0 + G : nchunks;
  return s;
}

__global__ __launch_bounds__(NT) void ret_seg_state(const uint16_t* __restrict__ k,
                                                    const uint16_t* __restrict__ v,
                                                    const float* __restrict__ gamma, int H,
                                                    int64_t T, int nseg, int G,
                                                    float* __restrict__ ws) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int64_t nchunks = T / CH;
  const SegGeom sg = seg_geom(nseg, G, nchunks);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const float lg = __log2f(gamma[sg.bh % H]);
  const float gC = __builtin_amdgcn_exp2f((float)CH * lg);
  k += sg.bh * T * HD;
  v += sg.bh * T * HD;
  f32x16 S[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) S[cb][r] = 0.f;
  ChunkRegs cur, nxt;
  if (sg.c0 < sg.c1) load_kv(cur, k, v, sg.c0 * CH, tid);
  for (int64_t ci = sg.c0; ci < sg.c1; ++ci) {
    store_kv<false>(lds, cur, lg, tid);
    __syncthreads();
    if (ci + 1 < sg.c1) load_kv(nxt, k, v, (ci + 1) * CH, tid);
    state_update(S, lds, gC, wave, l32, g);
    __syncthreads();
    if (ci + 1 < sg.c1) cur = nxt;
  }
  float* E = ws + (sg.bh * nseg + sg.seg) * (int64_t)(HD * HD);
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) E[(32 * wave + acc_row(r, g)) * HD + 32 * cb + l32] = S[cb][r];
}

// In place: ws[bh][s] := state entering segment s.
__global__ __launch_bounds__(NT) void ret_seg_carry(const float* __restrict__ gamma, int H,
                                                    int nseg, int G, float* __restrict__ ws) {
  const int64_t bh = blockIdx.y;
  const int e = blockIdx.x * NT + threadIdx.x;  // element of the 128x128 state
  const float gSeg = __builtin_amdgcn_exp2f((float)(CH * G) * __log2f(gamma[bh % H]));
  float cin = 0.f;
  float* base = ws + bh * nseg * (int64_t)(HD * HD) + e;
  for (int s = 0; s < nseg; ++s) {
    const float es = base[(int64_t)s * HD * HD];
    base[(int64_t)s * HD * HD] = cin;
    cin = gSeg * cin + es;
  }
}

__global__ __launch_bounds__(NT) void ret_seg_out(const uint16_t* __restrict__ q,
                                                  const uint16_t* __restrict__ k,
                                                  const uint16_t* __restrict__ v,
                                                  const float* __restrict__ gamma, int H,
                                                  int64_t T, int nseg, int G, float scale,
                                                  int zero_start, const float* __restrict__ ws,
                                                  uint16_t* __restrict__ o) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int64_t nchunks = T / CH;
  const SegGeom sg = seg_geom(nseg, G, nchunks);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int qb = wave & 1, dh = wave >> 1;
  const float lg = __log2f(gamma[sg.bh % H]);
  const float gC = __builtin_amdgcn_exp2f((float)CH * lg);
  q += sg.bh * T * HD;
  k += sg.bh * T * HD;
  v += sg.bh * T * HD;
  o += sg.bh * T * HD;

  // Start state of this segment.
  f32x16 S[4];
  const float* Sst = ws + (sg.bh * nseg + sg.seg) * (int64_t)(HD * HD);
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      S[cb][r] = zero_start ? 0.f : Sst[(32 * wave + acc_row(r, g)) * HD + 32 * cb + l32];

  const int qi = 32 * qb + l32;  // this lane's query within the chunk
  const float qrow_decay = __builtin_amdgcn_exp2f((float)qi * lg);
  ChunkRegs cur, nxt;
  bf16x8 qf[HD / 16], qn[HD / 16];
  auto load_q = [&](bf16x8 (&dst)[HD / 16], int64_t t0) {
#pragma unroll
    for (int j = 0; j < HD / 16; ++j)
      dst[j] = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const u32x4*>(q + (t0 + qi) * HD + 16 * j + 8 * g));
  };
  if (sg.c0 < sg.c1) {
    load_kv(cur, k, v, sg.c0 * CH, tid);
    load_q(qf, sg.c0 * CH);
  }
  for (int64_t ci = sg.c0; ci < sg.c1; ++ci) {
    const int64_t t0 = ci * CH;
    // 1. tiles + bf16 copy of the state entering this chunk (Sᵀ[dv][dk]).
    store_kv<true>(lds, cur, lg, tid);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int dv = 32 * cb + l32;
        const int dk = 32 * wave + 8 * rg + 4 * g;
        const u32x2 w = u32x2{pack_bf16x2(S[cb][4 * rg], S[cb][4 * rg + 1]),
                              pack_bf16x2(S[cb][4 * rg + 2], S[cb][4 * rg + 3])};
        *reinterpret_cast<u32x2*>(lds + OFF_ST + st_off(dv, dk >> 3) + (dk & 7)) = w;
      }
    }
    __syncthreads();
    if (ci + 1 < sg.c1) {
      load_kv(nxt, k, v, t0 + CH, tid);
      load_q(qn, t0 + CH);
    }
    // 2. sᵀ = k qᵀ over both key blocks of this wave's query block.
    f32x16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
    for (int j = 0; j < HD / 16; ++j)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(lds + OFF_K + k_off(32 * kb + l32, 2 * j + g));
        sacc[kb] = mfma32x32x16(a, qf[j], sacc[kb]);
      }
    // 3. Pᵀ = sᵀ ⊙ Dᵀ, Dᵀ[key][q] = γ^(q-key) for key <= q.
    bf16x8 pf[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 32 * kb + acc_row(r, g);
        const float dcy = key <= qi ? __builtin_amdgcn_exp2f((float)(qi - key) * lg) : 0.f;
        pf[kb][r >> 3][r & 7] = static_cast<__bf16>(sacc[kb][r] * dcy);
      }
    // 4./5. intraᵀ and crossᵀ for value rows 64*dh .. +64.
    f32x16 oacc[2], cacc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[i][r] = cacc[i][r] = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int dv = 64 * dh + 32 * i + l32;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int unit = 8 * kb + 4 * u + g;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(lds + OFF_VT + t_off(dv, unit));
          const u32x2 hi = *reinterpret_cast<const u32x2*>(lds + OFF_VT + t_off(dv, unit + 2));
          oacc[i] = mfma32x32x16(__builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]}),
                                 pf[kb][u], oacc[i]);
        }
#pragma unroll
      for (int j = 0; j < HD / 16; ++j) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(lds + OFF_ST + st_off(dv, 2 * j + g));
        cacc[i] = mfma32x32x16(a, qf[j], cacc[i]);
      }
    }
    // 6. o[t0 + qi][dv] = scale * (intra + γ^qi cross)
    uint16_t* orow = o + (t0 + qi) * HD;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int dv = 64 * dh + 32 * i + 8 * rg + 4 * g;
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = scale * (oacc[i][4 * rg + e] + qrow_decay * cacc[i][4 * rg + e]);
        *reinterpret_cast<u32x2*>(orow + dv) = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
      }
    // 7. state update with this chunk.
    state_update(S, lds, gC, wave, l32, g);
    __syncthreads();
    if (ci + 1 < sg.c1) {
      cur = nxt;
#pragma unroll
      for (int j = 0; j < HD / 16; ++j) qf[j] = qn[j];
    }
  }
}

struct RetPlan {
  int nseg, G;
};

RetPlan ret_plan(int64_t B, int64_t H, int64_t T) {
  const int64_t bh = B * H, nchunks = T / CH;
  int64_t nseg = (512 + bh - 1) / (bh > 0 ? bh : 1);
  if (nseg < 1) nseg = 1;
  if (nseg > nchunks) nseg = nchunks > 0 ? nchunks : 1;
  int64_t G = (nchunks + nseg - 1) / nseg;
  if (G < 1) G = 1;
  nseg = (nchunks + G - 1) / G;
  if (nseg < 1) nseg = 1;
  return RetPlan{(int)nseg, (int)G};
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int64_t catopt_hip_retention_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t d,
                                                        int64_t chunk) {
  if (B < 0 || H < 0 || T < 0 || d != HD || chunk != CH) return -1;
  const RetPlan p = ret_plan(B, H, T);
  return B * H * (int64_t)p.nseg * HD * HD * (int64_t)sizeof(float);
}

extern "C" int32_t catopt_hip_retention_fwd(int32_t dtype, int64_t B, int64_t H, int64_t T,
                                            int64_t d, int64_t chunk, const void* q, const void* k,
                                            const void* v, const float* gamma, float scale, void* o,
                                            void* workspace, int64_t workspace_bytes,
                                            void* stream) {
  if (B < 0 || H < 0 || T < 0) return CATOPT_E_INVAL;
  if (dtype != CATOPT_BF16 || d != HD || chunk != CH) return CATOPT_E_UNSUPPORTED;
  if (T % CH != 0) return CATOPT_E_UNSUPPORTED;
  if (B == 0 || H == 0 || T == 0) return CATOPT_OK;
  if (!q || !k || !v || !gamma || !o) return CATOPT_E_INVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return CATOPT_E_INVAL;
  if (B * H > 0x7fffffffLL / 64) return CATOPT_E_UNSUPPORTED;
  const int64_t need = catopt_hip_retention_workspace_bytes(B, H, T, d, chunk);
  if (!workspace || workspace_bytes < need) return CATOPT_E_WORKSPACE;
  static bool attr_done = false;
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&ret_seg_state),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(&ret_seg_out),
                              hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (e != hipSuccess) return set_hip_error(e);
    attr_done = true;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const RetPlan p = ret_plan(B, H, T);
  const int64_t blocks = B * H * p.nseg;
  auto qp = static_cast<const uint16_t*>(q);
  auto kp = static_cast<const uint16_t*>(k);
  auto vp = static_cast<const uint16_t*>(v);
  float* ws = static_cast<float*>(workspace);
  // A single segment starts from the zero state and needs no carry pass.
  if (p.nseg > 1) {
    ret_seg_state<<<dim3((uint32_t)blocks), dim3(NT), LDS_BYTES, s>>>(kp, vp, gamma, (int)H, T, p.nseg, p.G, ws);
    CATOPT_LAUNCH_CHECK();
    ret_seg_carry<<<dim3(HD * HD / NT, (uint32_t)(B * H)), dim3(NT), 0, s>>>(gamma, (int)H, p.nseg, p.G, ws);
    CATOPT_LAUNCH_CHECK();
  }
  ret_seg_out<<<dim3((uint32_t)blocks), dim3(NT), LDS_BYTES, s>>>(
      qp, kp, vp, gamma, (int)H, T, p.nseg, p.G, scale, p.nseg > 1 ? 0 : 1, ws,
      static_cast<uint16_t*>(o));
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}
