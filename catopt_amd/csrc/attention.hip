// Online-softmax attention forward for gfx950 (bf16 in, fp32 math).
//
// Transposed FlashAttention formulation chosen for the 32x32 MFMA layouts:
//
//   Sᵀ = K · Qᵀ      A = K tile from LDS (key rows, d contiguous),
//                    B = Q fragments held in registers for the whole loop.
//   Oᵀ += Vᵀ · Pᵀ    A = Vᵀ from LDS, B = P straight from the Sᵀ
//                    accumulator registers (converted to bf16).
//
// In both products the accumulator's column is the query, so every lane
// owns exactly one query: the running max m, the denominator l and the
// rescale of Oᵀ are lane-local, and only one cross-half shuffle per KV tile
// (the row max) is needed.  Feeding P from the accumulator works because
// the MFMA's k index is only a summation order: the PV product pairs
// accumulator register r of half g with key 8*(r/4) + 4*g + r%4, and Vᵀ is
// read from LDS with the same key permutation (two 8-byte runs per lane).
//
// Work split: one workgroup = 4 waves = 128 queries of one (b, h); each
// wave 32 queries.  KV tiles of 64 keys are double buffered in LDS: K as
// [key][d] with 16-byte chunks XOR-swizzled by the key, V transposed to
// [d][key] with 8-byte key groups XOR-swizzled by d/2, both conflict-free
// for the fragment reads.  Causal grids launch the longest query tiles
// first.  Softmax runs in the exp2 domain with scale·log2(e) folded in.
#include "common.hpp"

namespace catopt {
namespace {

constexpr int NT = 256;  // 4 waves
constexpr int QT = 128;  // queries per workgroup
constexpr int KVB = 64;  // keys per KV tile

template <int D>
struct AttnLds {
  static constexpr int K_ELEMS = KVB * D;
  static constexpr int V_ELEMS = D * KVB;
  static constexpr int STAGE = K_ELEMS + V_ELEMS;
  static constexpr int BYTES = 2 * STAGE * 2;
  static constexpr int KCH = D / 8;  // 16-byte chunks per K row
};

template <int D>
__device__ __forceinline__ int k_off(int key, int chunk) {
  return key * D + ((chunk ^ (key & (AttnLds<D>::KCH - 1))) << 3);
}
// Vᵀ row d holds 64 keys = 16 units of 4 keys (8 bytes).
__device__ __forceinline__ int vt_off(int d, int unit) {
  return d * KVB + ((unit ^ ((d >> 1) & 15)) << 2);
}

template <int D, int MASK>
__global__ __launch_bounds__(NT) void attn_fwd_kernel(
    const uint16_t* __restrict__ q, int64_t qsb, int64_t qsh, int64_t qst,
    const uint16_t* __restrict__ k, int64_t ksb, int64_t ksh, int64_t kst,
    const uint16_t* __restrict__ v, int64_t vsb, int64_t vsh, int64_t vst,
    uint16_t* __restrict__ o, int64_t osb, int64_t osh, int64_t ost, float* __restrict__ m_out,
    float* __restrict__ l_out, int H, int Tq, int Tk, float scale_log2, int64_t causal_off,
    const uint8_t* __restrict__ mask, int64_t mask_ld, int normalize) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  using L = AttnLds<D>;
  const int nqt = gridDim.x;
  const int qt = (MASK == CATOPT_MASK_CAUSAL) ? (nqt - 1 - (int)blockIdx.x) : (int)blockIdx.x;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  q += b * qsb + h * qsh;
  k += b * ksb + h * ksh;
  v += b * vsb + h * vsh;
  o += b * osb + h * osh;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = qt * QT;
  const int qrow = q0 + wave * 32 + l32;
  const bool qok = qrow < Tq;

  // Q fragments (MFMA B operand): Q[qrow][16j + 8g .. +8]
  bf16x8 qf[D / 16];
#pragma unroll
  for (int j = 0; j < D / 16; ++j) {
    u32x4 t = u32x4{0, 0, 0, 0};
    if (qok) t = *reinterpret_cast<const u32x4*>(q + (int64_t)qrow * qst + 16 * j + 8 * g);
    qf[j] = __builtin_bit_cast(bf16x8, t);
  }

  f32x16 oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[i][r] = 0.f;
  float m_run = -__builtin_inff();
  float l_run = 0.f;

  int64_t kv_end = Tk;
  if (MASK == CATOPT_MASK_CAUSAL) {
    const int64_t lim = (int64_t)q0 + QT + causal_off;  // last query's last key + 1
    kv_end = lim < 0 ? 0 : (lim < Tk ? lim : Tk);
  }
  const int nkv = (int)((kv_end + KVB - 1) / KVB);

  // Tile loaders: K rows (16-byte chunks), V as 4-key x 8-d blocks.
  constexpr int K_UNITS = KVB * L::KCH;            // 16-byte chunks per K tile
  constexpr int K_PER_T = K_UNITS / NT;
  constexpr int V_UNITS = (KVB / 4) * (D / 8);     // 4-key x 8-d blocks per V tile
  constexpr int V_PER_T = (V_UNITS + NT - 1) / NT;
  u32x4 rk[K_PER_T];
  u32x4 rv[V_PER_T][4];

  auto gload = [&](int kvt) {
    const int kv0 = kvt * KVB;
#pragma unroll
    for (int i = 0; i < K_PER_T; ++i) {
      const int u = tid + i * NT;
      const int key = u / L::KCH, ch = u % L::KCH;
      const int gk = kv0 + key;
      rk[i] = gk < Tk ? *reinterpret_cast<const u32x4*>(k + (int64_t)gk * kst + ch * 8)
                      : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < V_PER_T; ++i) {
      const int u = tid + i * NT;
      const int c = u % (D / 8), kk = u / (D / 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int gk = kv0 + 4 * kk + e;
        rv[i][e] = (u < V_UNITS && gk < Tk)
                       ? *reinterpret_cast<const u32x4*>(v + (int64_t)gk * vst + c * 8)
                       : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto sstore = [&](int stage) {
    uint16_t* Ks = lds + stage * L::STAGE;
    uint16_t* Vt = Ks + L::K_ELEMS;
#pragma unroll
    for (int i = 0; i < K_PER_T; ++i) {
      const int u = tid + i * NT;
      *reinterpret_cast<u32x4*>(Ks + k_off<D>(u / L::KCH, u % L::KCH)) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < V_PER_T; ++i) {
      const int u = tid + i * NT;
      if (u >= V_UNITS) continue;
      const int c = u % (D / 8), kk = u / (D / 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // element e of the 8-d chunk: bf16 (e&1) of dword (e>>1), for 4 keys
        const int sh = (e & 1) * 16, w = e >> 1;
        const uint32_t k0 = (rv[i][0][w] >> sh) & 0xffffu, k1 = (rv[i][1][w] >> sh) & 0xffffu;
        const uint32_t k2 = (rv[i][2][w] >> sh) & 0xffffu, k3 = (rv[i][3][w] >> sh) & 0xffffu;
        *reinterpret_cast<u32x2*>(Vt + vt_off(c * 8 + e, kk)) = u32x2{k0 | (k1 << 16), k2 | (k3 << 16)};
      }
    }
  };

  if (nkv > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  for (int kvt = 0; kvt < nkv; ++kvt) {
    const int cur = kvt & 1;
    if (kvt + 1 < nkv) gload(kvt + 1);
    const uint16_t* Ks = lds + cur * L::STAGE;
    const uint16_t* Vt = Ks + L::K_ELEMS;
    const int kv0 = kvt * KVB;

    // Sᵀ tile: keys 32*kb + acc_row(r, g), query = this lane's.
    f32x16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(Ks + k_off<D>(32 * kb + l32, 2 * j + g));
        sacc[kb] = mfma32x32x16(a, qf[j], sacc[kb]);
      }
    }

    float mloc = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + 32 * kb + acc_row(r, g);
        float t = sacc[kb][r] * scale_log2;
        bool keep = key < Tk;
        if (MASK == CATOPT_MASK_CAUSAL) keep = keep && (int64_t)key <= (int64_t)qrow + causal_off;
        if (MASK == CATOPT_MASK_BOOL) keep = keep && qok && mask[(int64_t)qrow * mask_ld + key] != 0;
        t = keep ? t : -__builtin_inff();
        sacc[kb][r] = t;
        mloc = fmaxf(mloc, t);
      }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float lsum = 0.f;
    bf16x8 pf[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(sacc[kb][r] - m_use);
        lsum += p;
        pf[kb][r >> 3][r & 7] = static_cast<__bf16>(p);
      }
    }
    l_run = l_run * alpha + lsum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int unit = 8 * kb + 4 * u + g;
          const int d = 32 * db + l32;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(Vt + vt_off(d, unit));
          const u32x2 hi = *reinterpret_cast<const u32x2*>(Vt + vt_off(d, unit + 2));
          const bf16x8 a = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
          oacc[db] = mfma32x32x16(a, pf[kb][u], oacc[db]);
        }
      }
    }

    if (kvt + 1 < nkv) sstore(cur ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (!qok) return;
  const float inv = normalize ? 1.0f / l_tot : 1.0f;  // l_tot == 0 -> inf; 0 * inf = NaN (om_apply)
  uint16_t* orow = o + (int64_t)qrow * ost;
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int d = 32 * db + 8 * rg + 4 * g;
      float x0 = oacc[db][4 * rg + 0], x1 = oacc[db][4 * rg + 1];
      float x2 = oacc[db][4 * rg + 2], x3 = oacc[db][4 * rg + 3];
      if (normalize) {
        if (l_tot == 0.f) {
          x0 = x1 = x2 = x3 = __builtin_nanf("");
        } else {
          x0 *= inv; x1 *= inv; x2 *= inv; x3 *= inv;
        }
      }
      *reinterpret_cast<u32x2*>(orow + d) = u32x2{pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)};
    }
  }
  if (g == 0) {
    const int64_t mi = (b * H + h) * (int64_t)Tq + qrow;
    if (m_out) m_out[mi] = m_run * 0.69314718055994531f;  // back to natural-log units
    if (l_out) l_out[mi] = l_tot;
  }
}

template <int D, int MASK>
int32_t attn_launch(const uint16_t* q, const int64_t* qs, const uint16_t* k, const int64_t* ks,
                    const uint16_t* v, const int64_t* vs, uint16_t* o, const int64_t* os,
                    float* m_out, float* l_out, int64_t B, int64_t H, int64_t Tq, int64_t Tk,
                    float scale, int64_t causal_off, const uint8_t* mask, int64_t mask_ld,
                    int normalize, hipStream_t s) {
  static bool attr_done = false;
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_fwd_kernel<D, MASK>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, AttnLds<D>::BYTES);
    if (e != hipSuccess) return set_hip_error(e);
    attr_done = true;
  }
  const int64_t nqt = (Tq + QT - 1) / QT;
  const float scale_log2 = scale * 1.4426950408889634f;
  attn_fwd_kernel<D, MASK><<<dim3((uint32_t)nqt, (uint32_t)H, (uint32_t)B), dim3(NT), AttnLds<D>::BYTES, s>>>(
      q, qs[0], qs[1], qs[2], k, ks[0], ks[1], ks[2], v, vs[0], vs[1], vs[2], o, os[0], os[1],
      os[2], m_out, l_out, (int)H, (int)Tq, (int)Tk, scale_log2, causal_off, mask, mask_ld,
      normalize);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

template <int D>
int32_t attn_dispatch_mask(int32_t mode, const uint16_t* q, const int64_t* qs, const uint16_t* k,
                           const int64_t* ks, const uint16_t* v, const int64_t* vs, uint16_t* o,
                           const int64_t* os, float* m_out, float* l_out, int64_t B, int64_t H,
                           int64_t Tq, int64_t Tk, float scale, int64_t causal_off,
                           const uint8_t* mask, int64_t mask_ld, int normalize, hipStream_t s) {
  switch (mode) {
    case CATOPT_MASK_NONE:
      return attn_launch<D, CATOPT_MASK_NONE>(q, qs, k, ks, v, vs, o, os, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask, mask_ld, normalize, s);
    case CATOPT_MASK_CAUSAL:
      return attn_launch<D, CATOPT_MASK_CAUSAL>(q, qs, k, ks, v, vs, o, os, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask, mask_ld, normalize, s);
    case CATOPT_MASK_BOOL:
      return attn_launch<D, CATOPT_MASK_BOOL>(q, qs, k, ks, v, vs, o, os, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask, mask_ld, normalize, s);
    default:
      return CATOPT_E_INVAL;
  }
}

bool strides_ok(const int64_t* s) {
  return s && s[0] >= 0 && s[1] >= 0 && s[2] >= 0 && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0;
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int32_t catopt_hip_attn_fwd(int32_t dtype, int64_t B, int64_t H, int64_t Tq,
                                       int64_t Tk, int64_t d, int64_t dv, const void* q,
                                       const int64_t* q_strides, const void* k,
                                       const int64_t* k_strides, const void* v,
                                       const int64_t* v_strides, float scale, int32_t mask_mode,
                                       int64_t causal_off, const uint8_t* mask, int64_t mask_ld,
                                       int32_t normalize, void* o, const int64_t* o_strides,
                                       float* m_out, float* l_out, void* stream) {
  if (B < 0 || H < 0 || Tq < 0 || Tk < 0) return CATOPT_E_INVAL;
  if (mask_mode < CATOPT_MASK_NONE || mask_mode > CATOPT_MASK_BOOL) return CATOPT_E_INVAL;
  if (dtype != CATOPT_BF16) return CATOPT_E_UNSUPPORTED;
  if (d != dv || (d != 128 && d != 64)) return CATOPT_E_UNSUPPORTED;
  if (B == 0 || H == 0 || Tq == 0) return CATOPT_OK;
  if (!q || !k || !v || !o) return CATOPT_E_INVAL;
  if (!strides_ok(q_strides) || !strides_ok(k_strides) || !strides_ok(v_strides) ||
      !strides_ok(o_strides))
    return CATOPT_E_INVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return CATOPT_E_INVAL;
  if (mask_mode == CATOPT_MASK_BOOL && (!mask || mask_ld < Tk)) return CATOPT_E_INVAL;
  if (Tq > 0x7fffffffLL || Tk > 0x7fffffffLL || H > 65535 || B > 65535) return CATOPT_E_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto qp = static_cast<const uint16_t*>(q);
  auto kp = static_cast<const uint16_t*>(k);
  auto vp = static_cast<const uint16_t*>(v);
  auto op = static_cast<uint16_t*>(o);
  if (d == 128)
    return attn_dispatch_mask<128>(mask_mode, qp, q_strides, kp, k_strides, vp, v_strides, op,
                                   o_strides, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask,
                                   mask_ld, normalize, s);
  return attn_dispatch_mask<64>(mask_mode, qp, q_strides, kp, k_strides, vp, v_strides, op,
                                o_strides, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask,
                                mask_ld, normalize, s);
}
