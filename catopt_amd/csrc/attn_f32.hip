// fp32 attention carrier on gfx950 fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
//   s = scale · q kᵀ,   m = rowmax(s),   l = Σ_k exp(s − m),   a = Σ_k exp(s − m) v_k
//
// The om element of a score block (the (m, l, a) triple of om_elem), for
// fp32 operands and a value width dv independent of the key width dk: the
// deferred-affine attention leaves carry the two numerator parts [fa | fb]
// as one value block of width 2d (d·i + d for the dense fibre).  Scores,
// exponentials and the numerator never leave the chip.
//
// Transposed layout, as in the bf16 kernel (attention.hip): Sᵀ = K Qᵀ and
// Oᵀ += Vᵀ Pᵀ, so the accumulator column is the query and a lane owns one
// query: lane l holds rows (keys) 8·(r/4) + 4·(l/32) + r%4 of column l%32 in
// register r.  The running max, the denominator and the rescale of Oᵀ are
// lane-local plus one exchange between the two lane halves.  Pᵀ feeds the
// PV product from the Sᵀ accumulator: k-step t of that product pairs each
// lane half with its own register t (the MFMA's k index is a summation
// order), and the A operand reads the matching V row for each half.
//
// Work split: a workgroup is 4 waves x 32 queries; KV tiles of 32 keys are
// staged in LDS (K rows padded to dk + 2 floats, V rows to 32·DVB + 8, which
// keeps the column reads of K and the two half-rows of V on distinct banks).
// The max is moved eagerly (every tile that raises it rescales Oᵀ and l), so
// the emitted m is the true row max; a row with no finite score keeps m = −∞
// and l = 0, a = 0 (the empty carrier).
//
// Mask modes (as the bf16 kernel's): causal (keep key j for query i iff
// j <= i + causal_off; tiles past a workgroup's last key are skipped), a
// uint8 keep-plane, or an fp32 additive bias plane added to the scaled score
// (scale·q·k + bias, as torch forms it); the planes are (Tq, Tk) with row
// stride mask_ld, shared over the batch.
#include "common.hpp"

namespace catopt {
namespace {

constexpr int kWaves = 4, kNT = 64 * kWaves, kQT = 32 * kWaves, kKT = 32;

__device__ __forceinline__ f32x16 mfma_f32_32x32x2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int DK, int DVB>
struct CarrierLds {
  static constexpr int KST = DK + 2;            // K row stride (floats)
  static constexpr int VST = 32 * DVB + 8;      // V row stride (floats)
  static constexpr int BYTES = (kKT * KST + kKT * VST) * 4;
};

template <int DK, int DVB, int MASK>
__global__ __launch_bounds__(kNT) void attn_carrier_f32(
    const float* __restrict__ q, int64_t q_sb, int64_t ldq, const float* __restrict__ k, int64_t k_sb,
    int64_t ldk, const float* __restrict__ v, int64_t v_sb, int64_t ldv, float* __restrict__ m_out,
    float* __restrict__ l_out, float* __restrict__ num, int64_t n_sb, int64_t ldn, int Tq, int Tk, int dk,
    int dv, float scale, int64_t causal_off, const void* __restrict__ mask, int64_t mask_ld) {
  using L = CarrierLds<DK, DVB>;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Ks = smem;
  float* Vs = smem + kKT * L::KST;
  const int64_t bz = blockIdx.y;
  q += bz * q_sb;
  k += bz * k_sb;
  v += bz * v_sb;
  num += bz * n_sb;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int qrow = blockIdx.x * kQT + wave * 32 + l32;
  const bool qok = qrow < Tq;
  constexpr float c = 1.4426950408889634f;  // exp2 domain: exp(x) = exp2(x·log2 e)

  // Q as the B operand of Sᵀ = K Qᵀ: k-step j takes k index 2j + half.
  float qreg[DK / 2];
#pragma unroll
  for (int j = 0; j < DK / 2; ++j) {
    const int kk = 2 * j + g;
    qreg[j] = (qok && kk < dk) ? q[(int64_t)qrow * ldq + kk] : 0.f;
  }

  f32x16 oacc[DVB];
#pragma unroll
  for (int db = 0; db < DVB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_run = -__builtin_inff(), l_run = 0.f;

  // Tile staging: each thread moves KPT K and VPT V elements per tile.  The
  // next tile's elements are loaded into registers before this tile's
  // products and written to LDS after them, so the loads' latency hides
  // behind the MFMAs.  Elements past Tk / dk / dv are zero.
  constexpr int KPT = kKT * DK / kNT, VPT = kKT * 32 * DVB / kNT;
  // (the widest variants keep no prefetch: its registers would spill)
  constexpr bool PF = KPT + VPT <= 24;
  float kreg[KPT], vreg[VPT];
  auto load_tile = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int e = tid + i * kNT, r = e / DK, cc = e % DK, key = kv0 + r;
      kreg[i] = (key < Tk && cc < dk) ? k[(int64_t)key * ldk + cc] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = tid + i * kNT, r = e / (32 * DVB), cc = e % (32 * DVB), key = kv0 + r;
      vreg[i] = (key < Tk && cc < dv) ? v[(int64_t)key * ldv + cc] : 0.f;
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int e = tid + i * kNT;
      Ks[(e / DK) * L::KST + e % DK] = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = tid + i * kNT;
      Vs[(e / (32 * DVB)) * L::VST + e % (32 * DVB)] = vreg[i];
    }
  };

  // staging without the register round trip (variants with no prefetch)
  auto copy_tile = [&](int kv0) {
    for (int e = tid; e < kKT * DK; e += kNT) {
      const int r = e / DK, cc = e % DK, key = kv0 + r;
      Ks[r * L::KST + cc] = (key < Tk && cc < dk) ? k[(int64_t)key * ldk + cc] : 0.f;
    }
    for (int e = tid; e < kKT * 32 * DVB; e += kNT) {
      const int r = e / (32 * DVB), cc = e % (32 * DVB), key = kv0 + r;
      Vs[r * L::VST + cc] = (key < Tk && cc < dv) ? v[(int64_t)key * ldv + cc] : 0.f;
    }
  };

  int ntiles = (Tk + kKT - 1) / kKT;
  if (MASK == CATOPT_MASK_CAUSAL) {  // keys past the workgroup's last query + causal_off are masked
    const int64_t lim = (int64_t)blockIdx.x * kQT + kQT + causal_off;
    const int64_t nt = lim <= 0 ? 0 : (lim + kKT - 1) / kKT;
    if (nt < ntiles) ntiles = (int)nt;
  }
  if (ntiles > 0) {
    if (PF) {
      load_tile(0);
      store_tile();
    } else {
      copy_tile(0);
    }
    __syncthreads();
  }
  for (int t = 0; t < ntiles; ++t) {
    const int kv0 = t * kKT;
    if (PF && t + 1 < ntiles) load_tile(kv0 + kKT);

    // ---- Sᵀ = K Qᵀ (32 keys x 32 queries per wave)
    f32x16 sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
#pragma unroll
    for (int j = 0; j < DK / 2; ++j) sacc = mfma_f32_32x32x2(Ks[l32 * L::KST + 2 * j + g], qreg[j], sacc);

    // ---- online softmax over this tile's keys (eager max), on the scaled
    // score (a negative scale turns the raw minimum into the max)
    float tmax = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kv0 + 8 * (r >> 2) + 4 * g + (r & 3);
      bool keep = key < Tk;
      float add = 0.f;
      if (MASK == CATOPT_MASK_CAUSAL) keep = keep && (int64_t)key <= (int64_t)qrow + causal_off;
      if (MASK == CATOPT_MASK_BOOL || MASK == CATOPT_MASK_BIAS) {
        // the plane is read at a clamped, always-valid index; rows past Tq
        // are never stored
        const int64_t mi = (int64_t)(qok ? qrow : Tq - 1) * mask_ld + (key < Tk ? key : Tk - 1);
        if (MASK == CATOPT_MASK_BOOL) keep = keep && static_cast<const uint8_t*>(mask)[mi] != 0;
        if (MASK == CATOPT_MASK_BIAS) add = static_cast<const float*>(mask)[mi];
      }
      sacc[r] = keep ? __builtin_fmaf(sacc[r], scale, add) : -__builtin_inff();
      tmax = fmaxf(tmax, sacc[r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    float p[16];
    if (m_new == -__builtin_inff()) {
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = 0.f;
    } else {
      if (m_new > m_run) {
        const float alpha = (m_run == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f((m_run - m_new) * c);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DVB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
      }
      const float mc = m_new * c;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        // a bias can put scores near -FLT_MAX, where m·c overflows: the
        // difference s - m is exact there
        p[r] = MASK == CATOPT_MASK_BIAS ? __builtin_amdgcn_exp2f((sacc[r] - m_new) * c)
                                        : __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], c, -mc));  // exp2(-inf) = 0
        l_run += p[r];
      }
    }
    m_run = m_new;

    // ---- Oᵀ += Vᵀ Pᵀ: k-step r pairs each half with its own key 8(r/4) + 4g + r%4
#pragma unroll
    for (int db = 0; db < DVB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * g + (r & 3);
        oacc[db] = mfma_f32_32x32x2(Vs[key * L::VST + 32 * db + l32], p[r], oacc[db]);
      }
    }
    if (t + 1 < ntiles) {
      __syncthreads();  // every wave is done with this tile
      if (PF)
        store_tile();
      else
        copy_tile(kv0 + kKT);
      __syncthreads();
    }
  }

  // ---- carrier: m (scaled score), l over both halves, a relative to m
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (!qok) return;
  if (g == 0) {
    m_out[bz * Tq + qrow] = m_run;
    l_out[bz * Tq + qrow] = l_tot;
  }
  float* nrow = num + (int64_t)qrow * ldn;
#pragma unroll
  for (int db = 0; db < DVB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + 8 * (r >> 2) + 4 * g + (r & 3);
      if (d < dv) nrow[d] = oacc[db][r];
    }
  }
}

struct MaskArgs {
  int32_t mode;
  int64_t causal_off;
  const void* mask;
  int64_t ld;
};

template <int DK, int DVB>
int32_t carrier_launch(int64_t batch, int Tq, int Tk, int dk, int dv, const float* q, int64_t q_sb,
                       int64_t ldq, const float* k, int64_t k_sb, int64_t ldk, const float* v, int64_t v_sb,
                       int64_t ldv, float scale, float* m_out, float* l_out, float* num, int64_t n_sb,
                       int64_t ldn, const MaskArgs& ma, hipStream_t s) {
  using L = CarrierLds<DK, DVB>;
  const dim3 grid((uint32_t)((Tq + kQT - 1) / kQT), (uint32_t)batch);
#define CATOPT_CARRIER_MASK(M)                                                                                   attn_carrier_f32<DK, DVB, M><<<grid, dim3(kNT), L::BYTES, s>>>(q, q_sb, ldq, k, k_sb, ldk, v, v_sb, ldv,                                                                     m_out, l_out, num, n_sb, ldn, Tq, Tk, dk, dv,                                                                  scale, ma.causal_off, ma.mask, ma.ld)
  switch (ma.mode) {
    case CATOPT_MASK_NONE: CATOPT_CARRIER_MASK(CATOPT_MASK_NONE); break;
    case CATOPT_MASK_CAUSAL: CATOPT_CARRIER_MASK(CATOPT_MASK_CAUSAL); break;
    case CATOPT_MASK_BOOL: CATOPT_CARRIER_MASK(CATOPT_MASK_BOOL); break;
    case CATOPT_MASK_BIAS: CATOPT_CARRIER_MASK(CATOPT_MASK_BIAS); break;
    default: return CATOPT_E_INVAL;
  }
#undef CATOPT_CARRIER_MASK
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

template <int DK>
int32_t carrier_dv(int64_t batch, int Tq, int Tk, int dk, int dv, const float* q, int64_t q_sb, int64_t ldq,
                   const float* k, int64_t k_sb, int64_t ldk, const float* v, int64_t v_sb, int64_t ldv,
                   float scale, float* m_out, float* l_out, float* num, int64_t n_sb, int64_t ldn,
                   const MaskArgs& ma, hipStream_t s) {
  const int dvb = (dv + 31) / 32;
#define CATOPT_CARRIER(NB)                                                                                    \
  return carrier_launch<DK, NB>(batch, Tq, Tk, dk, dv, q, q_sb, ldq, k, k_sb, ldk, v, v_sb, ldv, scale, m_out, \
                                l_out, num, n_sb, ldn, ma, s)
  if (dvb <= 1) CATOPT_CARRIER(1);
  if (dvb <= 2) CATOPT_CARRIER(2);
  if (dvb <= 4) CATOPT_CARRIER(4);
  CATOPT_CARRIER(8);
#undef CATOPT_CARRIER
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int32_t catopt_hip_attn_carrier_f32_masked(
    int64_t batch, int64_t Tq, int64_t Tk, int64_t dk, int64_t dv, const float* q, int64_t q_sb, int64_t ldq,
    const float* k, int64_t k_sb, int64_t ldk, const float* v, int64_t v_sb, int64_t ldv, float scale,
    int32_t mask_mode, int64_t causal_off, const void* mask, int64_t mask_ld, float* m_out, float* l_out,
    float* num, int64_t num_sb, int64_t ldn, void* stream) {
  if (batch < 0 || Tq < 0 || Tk < 0 || dk < 1 || dv < 1) return CATOPT_E_INVAL;
  if (mask_mode < CATOPT_MASK_NONE || mask_mode > CATOPT_MASK_BIAS) return CATOPT_E_INVAL;
  if (dk > 128 || dv > 256) return CATOPT_E_UNSUPPORTED;
  if (batch == 0 || Tq == 0) return CATOPT_OK;
  if (!q || !m_out || !l_out || !num || (Tk > 0 && (!k || !v))) return CATOPT_E_INVAL;
  if (ldq < dk || ldk < dk || ldv < dv || ldn < dv || q_sb < 0 || k_sb < 0 || v_sb < 0 || num_sb < 0)
    return CATOPT_E_INVAL;
  if ((mask_mode == CATOPT_MASK_BOOL || mask_mode == CATOPT_MASK_BIAS) && Tk > 0 && (!mask || mask_ld < Tk))
    return CATOPT_E_INVAL;
  if (mask_mode == CATOPT_MASK_BIAS && (reinterpret_cast<uintptr_t>(mask) & 3)) return CATOPT_E_INVAL;
  if (batch > 65535 || Tq > 0x7fffffffLL - kQT || Tk > 0x7fffffffLL - kKT) return CATOPT_E_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int iTq = (int)Tq, iTk = (int)Tk, idk = (int)dk, idv = (int)dv;
  const MaskArgs ma{mask_mode, causal_off, mask, mask_ld};
#define CATOPT_CARRIER_DK(D)                                                                             \
  return carrier_dv<D>(batch, iTq, iTk, idk, idv, q, q_sb, ldq, k, k_sb, ldk, v, v_sb, ldv, scale, m_out, \
                       l_out, num, num_sb, ldn, ma, s)
  if (dk <= 16) CATOPT_CARRIER_DK(16);
  if (dk <= 32) CATOPT_CARRIER_DK(32);
  if (dk <= 64) CATOPT_CARRIER_DK(64);
  CATOPT_CARRIER_DK(128);
#undef CATOPT_CARRIER_DK
}

extern "C" int32_t catopt_hip_attn_carrier_f32(int64_t batch, int64_t Tq, int64_t Tk, int64_t dk, int64_t dv,
                                               const float* q, int64_t q_sb, int64_t ldq, const float* k,
                                               int64_t k_sb, int64_t ldk, const float* v, int64_t v_sb,
                                               int64_t ldv, float scale, float* m_out, float* l_out, float* num,
                                               int64_t num_sb, int64_t ldn, void* stream) {
  return catopt_hip_attn_carrier_f32_masked(batch, Tq, Tk, dk, dv, q, q_sb, ldq, k, k_sb, ldk, v, v_sb, ldv,
                                            scale, CATOPT_MASK_NONE, 0, nullptr, 0, m_out, l_out, num, num_sb,
                                            ldn, stream);
}
