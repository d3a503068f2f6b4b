// Online-softmax attention forward for gfx950 (bf16 in, fp32 math).
//
// Transposed FlashAttention formulation for the 32x32x16 MFMA layouts:
//
//   Sᵀ = K · Qᵀ      A = K tile from LDS (key rows, d contiguous),
//                    B = Q fragments held in registers for the whole loop.
//   Oᵀ += Vᵀ · Pᵀ    A = Vᵀ read from the row-major V tile with the gfx950
//                    transposing LDS read (ds_read_b64_tr_b16),
//                    B = P straight from the Sᵀ accumulator (bf16).
//
// In both products the accumulator's column is the query, so every lane
// owns one query per 32-query block: the running max, the denominator and
// the rescale of Oᵀ are lane-local, and only one cross-half shuffle per KV
// tile is needed.  P feeds the PV product from the accumulator because the
// MFMA's k index is only a summation order: accumulator register r of half
// g holds key 8*(r/4) + 4*g + r%4, and the A operand is read with the same
// key permutation (two runs of four consecutive keys per lane, which is one
// transposing read each).
//
// Work split: one workgroup = 4 waves = 128 queries of one (b, h), 32 per
// wave (QB = 1).  That keeps a wave within 256 registers, so two waves share
// each SIMD and one's softmax overlaps the other's MFMAs; QB = 2 (each K / V
// fragment feeding two MFMAs) needs AGPRs and measured 1.33x slower, from
// accumulator copies between the register files.  KV tiles of 64 keys are
// double buffered in LDS and filled by direct global->LDS loads through
// buffer resources (no register staging; rows past the keys read as zeros);
// K rows are 256 bytes with the 16-byte chunk index XOR-swizzled by
// (key & 15), V rows with the transposing-read swizzle below.  Causal grids
// launch the longest query tiles first, skip tiles past each wave's last key
// and apply the mask only on diagonal tiles.
//
// Within a wave a tile runs as two key halves of 32, each its own online-
// softmax step, so that the exponentials of one half issue between the MFMAs
// of the other (the interleaving is fixed with sched_group_barrier).  On
// MI355X that and reading all of a tile's K fragments before its first MFMA
// each measured 1-2%; copies of the kernel with one part taken out put the
// rest of the time in no single place (tile loads 12%, K or V fragment reads
// 5-6% each, exponentials 4%, half the MFMAs 23%).  Two alternatives measured
// slower: 8-wave workgroups whose two wave groups alternate MFMA and softmax
// phases between barriers, as the GEMM's ping-pong does (5%: with one
// MFMA-issuing wave per SIMD the fragment reads, 1 KB per MFMA and half of it
// through the half-rate transposing read, no longer keep the MFMAs fed;
// with the softmax taken out that variant still ran 574 us at C3), and
// raising the wave priority around the MFMA blocks (1.5%).
//
// Softmax runs in the exp2 domain: p = exp2((s - m) * c), c = scale·log2(e).
// The running max is only moved (and Oᵀ, l rescaled) when a tile raises it
// by more than kLazy/c; between moves p ≤ 2^kLazy, exact in fp32 and
// bf16's exponent range, and a / l is unchanged.  The true row max is
// tracked separately so the emitted (m, l, a) carrier is the om_elem one.
#include <type_traits>

#include "common.hpp"
#include "attn_q64_loop.inc"

namespace catopt {
namespace {

constexpr int NT = 256;   // 4 waves
constexpr int QB = 1;               // 32-query blocks per wave (the tile loop assumes 1)
constexpr int QW = 32 * QB;         // queries per wave
constexpr int QT = 4 * QW;          // queries per workgroup
constexpr int KVB = 64;   // keys per KV tile
constexpr float kLazy = 8.0f;

typedef __attribute__((ext_vector_type(4))) short s16x4;

template <int D>
struct AttnLds {
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int CH = D / 8;                  // 16-byte chunks per row
  static constexpr int TILE_BYTES = KVB * ROW_BYTES;
  static constexpr int STAGE_BYTES = 2 * TILE_BYTES;  // K then V
  static constexpr int BYTES = 2 * STAGE_BYTES;
  static constexpr int SLOTS = KVB * CH;            // 16-byte slots per tile
  static constexpr int SLOTS_PER_THREAD = SLOTS / NT;
};

// Byte offset of (key, 16-byte chunk) inside a swizzled tile.
template <int D>
__device__ __forceinline__ int tile_off(int key, int chunk) {
  return key * AttnLds<D>::ROW_BYTES + ((chunk ^ (key & (AttnLds<D>::CH - 1) & 15)) << 4);
}

// V tiles use their own swizzle.  A transposing read of Vᵀ covers, per
// 32-lane pass, 4 consecutive keys x 4 adjacent 16-byte chunks; XOR-ing the
// chunk index with 4 * (the key's position among those 4, per 256-byte bank
// window) puts the 16 pieces in 16 different bank groups (the key-row
// swizzle above would put all 4 keys on the same 4 groups).
template <int D>
__device__ __forceinline__ int vswz(int key) {
  constexpr int R = 256 / AttnLds<D>::ROW_BYTES;  // tile rows per 256-byte bank window
  return 4 * ((key / R) & (4 / R - 1));
}
template <int D>
__device__ __forceinline__ int vtile_off(int key, int chunk) {
  return key * AttnLds<D>::ROW_BYTES + ((chunk ^ vswz<D>(key)) << 4);
}

// An empty asm use: the value must be computed before this point, which
// keeps the compiler from sinking its computation out of an interleaved
// region into a later block.
__device__ __forceinline__ void pin(const bf16x8& x) {
  asm volatile("" ::"v"(__builtin_bit_cast(u32x4, x)));
}
__device__ __forceinline__ void pin(float x) { asm volatile("" ::"v"(x)); }

__device__ __forceinline__ s16x4 ds_read_tr(const char* lds_base, int byte_off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds_base + byte_off));
}

// (head, query tile) of this workgroup in a 1-D grid of nqt x H x B tiles.
// Workgroups are dealt round robin over the 8 XCDs (linear id L runs on XCD
// L % 8).  Each XCD owns a contiguous range of heads, so that K and V of a
// head stay in one XCD's L2, and takes them in pairs of heads, each pair in
// query-tile order (qi = 0, the longest causal tile, of both heads first).
// Head by head left a tail of long tiles started late (about 10% of a
// causal launch at C3's shape); all of an XCD's heads in query-tile order
// kept 16 heads' K and V in flight and read 3.5x the algorithmic bytes from
// HBM.  Pairs keep both the tail and the traffic down.
__device__ __forceinline__ void tile_of_block(int nqt, int& bh, int& qi) {
  const int nblk = gridDim.x, nbh = nblk / nqt;
  if ((nblk & 7) == 0 && (nbh & 15) == 0) {
    const int hx = nbh >> 3, kk = blockIdx.x >> 3;
    const int pair = kk / (2 * nqt), w = kk - pair * 2 * nqt;
    qi = w >> 1;
    bh = (blockIdx.x & 7) * hx + 2 * pair + (w & 1);
  } else {
    int w = blockIdx.x;
    if ((nblk & 7) == 0) w = (w & 7) * (nblk >> 3) + (w >> 3);
    bh = w / nqt;
    qi = w - bh * nqt;
  }
}

template <int D, int MASK>
__global__ __launch_bounds__(NT, QB == 1 ? 2 : 1) void attn_fwd_kernel(
    const uint16_t* __restrict__ q, int64_t qsb, int64_t qsh, int64_t qst,
    const uint16_t* __restrict__ k, int64_t ksb, int64_t ksh, int64_t kst,
    const uint16_t* __restrict__ v, int64_t vsb, int64_t vsh, int64_t vst,
    uint16_t* __restrict__ o, int64_t osb, int64_t osh, int64_t ost, float* __restrict__ m_out,
    float* __restrict__ l_out, int H, int Tq, int Tk, float scale, int64_t causal_off,
    const void* __restrict__ mask, int64_t mask_ld, int normalize) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  using L = AttnLds<D>;
  const int nqt = (Tq + QT - 1) / QT;
  int bh, qi;
  tile_of_block(nqt, bh, qi);
  const int qt = (MASK == CATOPT_MASK_CAUSAL) ? (nqt - 1 - qi) : qi;
  const int64_t b = bh / H, h = bh - (int64_t)(bh / H) * H;
  q += b * qsb + h * qsh;
  k += b * ksb + h * ksh;
  v += b * vsb + h * vsh;
  o += b * osb + h * osh;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = qt * QT;
  const int qw0 = q0 + wave * QW;  // first query of this wave
  // Scores run in raw q·k units, scaled at the exponential by c.  The bias
  // mode instead forms torch's scaled score scale·q·k + bias in the mask
  // step (dividing the bias by the scale instead overflows a finfo.min
  // bias to -inf), and its exponentials use c = log2(e).
  constexpr bool kScaledScores = MASK == CATOPT_MASK_BIAS;
  const float c = kScaledScores ? 1.4426950408889634f : scale * 1.4426950408889634f;
  const float m_unit = kScaledScores ? 1.f : scale;  // natural-log units of the scaled score

  // Q fragments (MFMA B operand) for the wave's two 32-query blocks.
  bf16x8 qf[QB][D / 16];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qrow = qw0 + 32 * qb + l32;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      u32x4 t = u32x4{0, 0, 0, 0};
      if (qrow < Tq) t = *reinterpret_cast<const u32x4*>(q + (int64_t)qrow * qst + 16 * j + 8 * g);
      qf[qb][j] = __builtin_bit_cast(bf16x8, t);
    }
  }

  f32x16 oacc[D / 32][QB];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[i][qb][r] = 0.f;
  float m_run[QB], m_true[QB], l_run[QB];  // maxima in raw-score units
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = m_true[qb] = -__builtin_inff();
    l_run[qb] = 0.f;
  }

  int64_t kv_end = Tk, wave_end = Tk;
  if (MASK == CATOPT_MASK_CAUSAL) {
    const int64_t lim = (int64_t)q0 + QT + causal_off;
    kv_end = lim < 0 ? 0 : (lim < Tk ? lim : Tk);
    const int64_t wl = (int64_t)qw0 + QW + causal_off;
    wave_end = wl < 0 ? 0 : (wl < Tk ? wl : Tk);
  }
  const int nkv = (int)((kv_end + KVB - 1) / KVB);

  // Fill one stage: K and V tiles of keys [kv0, kv0 + 64) by direct
  // global->LDS loads through buffer resources over the tile's rows.  Each
  // thread owns SLOTS_PER_THREAD fixed 16-byte slots whose byte offsets
  // inside a tile are computed once (the host guarantees 64 rows of either
  // stride fit in 31 bits); rows past Tk lie outside the resource and read
  // as zeros, so a tail tile needs no clamping and its V rows past Tk are 0.
  // (literal array bounds: with a bound that depends on D the host pass
  // takes the arrays for variable-length ones and silently drops the
  // kernel's launch stub; 4 = SLOTS_PER_THREAD at D = 128, the largest)
  static_assert(AttnLds<D>::SLOTS_PER_THREAD <= 4, "slot arrays hold 4 entries");
  uint32_t t_koff[4], t_voff[4];
#pragma unroll
  for (int i = 0; i < L::SLOTS_PER_THREAD; ++i) {
    const int s = i * NT + wave * 64 + lane;
    const int row = s / L::CH, cp = s % L::CH;
    const int chunk = cp ^ (row & (L::CH - 1) & 15);
    const int vchunk = cp ^ vswz<D>(row);
    t_koff[i] = (uint32_t)(row * (int)kst + chunk * 8) * 2u;
    t_voff[i] = (uint32_t)(row * (int)vst + vchunk * 8) * 2u;
  }
  auto issue_tile = [&](int kvt, int stage) {
    const int kv0 = kvt * KVB;
    const int64_t rows = Tk - kv0 < KVB ? Tk - kv0 : KVB;
    const u32x4 kr = make_rsrc(k + (int64_t)kv0 * kst, (uint32_t)(((rows - 1) * kst + D) * 2));
    const u32x4 vr = make_rsrc(v + (int64_t)kv0 * vst, (uint32_t)(((rows - 1) * vst + D) * 2));
    const uint32_t sb = lds_u32(lds + stage * L::STAGE_BYTES) + wave * 64 * 16;
#pragma unroll
    for (int i = 0; i < L::SLOTS_PER_THREAD; ++i) {
      dma_buf(kr, t_koff[i], sb + i * NT * 16);
      dma_buf(vr, t_voff[i], sb + i * NT * 16 + L::TILE_BYTES);
    }
  };

  if (nkv > 0) {
    issue_tile(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // one KV tile; the stage is a compile-time constant (the loop below runs
  // the tiles in pairs), so every LDS fragment address is a loop-invariant
  // lane offset plus an immediate
  auto tile = [&](int kvt, auto stage_tag) {
    constexpr int cur = decltype(stage_tag)::value;
    if (kvt + 1 < nkv) issue_tile(kvt + 1, cur ^ 1);
    const char* Ks = lds + cur * L::STAGE_BYTES;
    const char* Vs = Ks + L::TILE_BYTES;
    const int kv0 = kvt * KVB;

    if (kv0 < wave_end) {
      // The tile runs as two key halves of 32 (kb = 0, 1), each its own
      // online-softmax step, so that the exponentials of one half issue
      // between the MFMAs of the other in one instruction stream:
      //   QK(0) | max(0) | QK(1) + exp(0) | max(1) | PV(0) + exp(1) | PV(1)
      // (+: interleaved by sched_group_barrier).  A move of the reference
      // max asked for by half 1 rescales Oᵀ after PV(0), whose probabilities
      // are relative to the previous reference, and before PV(1).
      bool need_mask = kv0 + KVB > Tk;
      if (MASK == CATOPT_MASK_CAUSAL) need_mask = need_mask || (int64_t)kv0 + KVB - 1 > (int64_t)qw0 + causal_off;
      if (MASK == CATOPT_MASK_BOOL || MASK == CATOPT_MASK_BIAS) need_mask = true;
      const int qrow = qw0 + l32;

      bf16x8 kf[2][D / 16], vf[2][D / 16];
      auto read_k = [&](int kb) {
#pragma unroll
        for (int j = 0; j < D / 16; ++j)
          kf[kb][j] = *reinterpret_cast<const bf16x8*>(Ks + tile_off<D>(32 * kb + l32, 2 * j + g));
      };
      // Vᵀ fragments of key half kb.  Lane: group G = lane / 16, j = lane %
      // 16 -> keys key0 + j / 4 and key0 + 8 + j / 4, d block 4 (j % 4).
      auto read_v = [&](int kb) {
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int G = lane >> 4, jj = lane & 15;
            const int key0 = 32 * kb + 16 * u + 4 * (G >> 1) + (jj >> 2);
            const int d = 32 * db + 16 * (G & 1) + 4 * (jj & 3);
            const int chunk = d >> 3, half = (d & 7) * 2;
            const s16x4 lo = ds_read_tr(Vs, vtile_off<D>(key0, chunk) + half);
            const s16x4 hi = ds_read_tr(Vs, vtile_off<D>(key0 + 8, chunk) + half);
            vf[kb][2 * db + u] = __builtin_bit_cast(
                bf16x8, u32x4{__builtin_bit_cast(u32x2, lo)[0], __builtin_bit_cast(u32x2, lo)[1],
                              __builtin_bit_cast(u32x2, hi)[0], __builtin_bit_cast(u32x2, hi)[1]});
          }
        }
      };
      // Sᵀ of key half kb (32 keys x 32 queries)
      auto qk = [&](int kb, f32x16& s) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
        for (int j = 0; j < D / 16; ++j) s = mfma32x32x16(kf[kb][j], qf[0][j], s);
      };
      // Oᵀ += Vᵀ Pᵀ over key half kb
      auto pv = [&](int kb, const bf16x8* p) {
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
          for (int u = 0; u < 2; ++u) oacc[db][0] = mfma32x32x16(vf[kb][2 * db + u], p[u], oacc[db][0]);
      };
      // mask (diagonal / tail / bool / bias tiles only), branch-free: every
      // lane evaluates every predicate (the mask byte is read at a clamped,
      // always-valid address) and the score is replaced by a select
      auto apply_mask = [&](int kb, f32x16& s) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + 32 * kb + acc_row(r, g);
          bool keep = key < Tk;
          if (MASK == CATOPT_MASK_CAUSAL) keep = keep & ((int64_t)key <= (int64_t)qrow + causal_off);
          float add = 0.f;
          if (MASK == CATOPT_MASK_BOOL || MASK == CATOPT_MASK_BIAS) {
            const int qc = qrow < Tq ? qrow : Tq - 1;
            const int kc = key < Tk ? key : Tk - 1;
            const int64_t mi = (int64_t)qc * mask_ld + kc;
            if (MASK == CATOPT_MASK_BOOL) keep = keep & (static_cast<const uint8_t*>(mask)[mi] != 0);
            if (MASK == CATOPT_MASK_BIAS) add = static_cast<const float*>(mask)[mi];
            keep = keep & (qrow < Tq);
          }
          if (kScaledScores)
            s[r] = keep ? __builtin_fmaf(s[r], scale, add) : -__builtin_inff();
          else
            s[r] = keep ? s[r] : -__builtin_inff();
        }
      };
      // row max of a half (both lane halves), the true max, and the lazy
      // move of the reference max; returns the factor for Oᵀ (1: no move)
      auto half_max = [&](const f32x16& s) -> float {
        float mt = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[r]);
        {  // max with the other lane half, on the VALU (an LDS shuffle would
           // wait behind the fragment reads in flight)
          const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mt),
                                                           __builtin_bit_cast(uint32_t, mt), false, false);
          mt = fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
        }
        m_true[0] = fmaxf(m_true[0], mt);
        // move the reference max only when this half exceeds it by kLazy (log2 units)
        float alpha = 1.f;
        if (__builtin_amdgcn_ballot_w64((mt - m_run[0]) * c > kLazy) != 0) {
          const float m_new = fmaxf(m_run[0], mt);
          alpha = (m_run[0] == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f((m_run[0] - m_new) * c);
          l_run[0] *= alpha;
          m_run[0] = m_new;
        }
        return alpha;
      };
      auto rescale = [&](float alpha) {
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][0][r] *= alpha;
      };
      // p = exp2(s c - m c) as the bf16 B operand of PV, and its row sum
      auto half_exp = [&](const f32x16& s, bf16x8* p) {
        const float mr = (m_run[0] == -__builtin_inff()) ? 0.f : m_run[0];
        const float mc = mr * c;
        float lsum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          // scaled scores may sit near -FLT_MAX (a finfo.min bias), where
          // s·c - m·c as one fma leaves m·c's rounding error (or overflow);
          // the difference s - m is exact there
          const float e = kScaledScores ? __builtin_amdgcn_exp2f((s[r] - mr) * c)
                                        : __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -mc));
          lsum += e;
          p[r >> 3][r & 7] = static_cast<__bf16>(e);
        }
        l_run[0] += lsum;
      };

      f32x16 s0, s1;
      bf16x8 p0[2], p1[2];
      read_k(0);
      read_k(1);
      qk(0, s0);
      if (need_mask) apply_mask(0, s0);
      const float a0 = half_max(s0);
      if (a0 != 1.f) rescale(a0);
      // QK(1) + exp(0), and the Vᵀ fragments of half 0
      __builtin_amdgcn_sched_barrier(0);
      qk(1, s1);
      half_exp(s0, p0);
      read_v(0);
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // VALU
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // DS read
      }
      pin(p0[0]);
      pin(p0[1]);
      pin(l_run[0]);
      __builtin_amdgcn_sched_barrier(0);
      if (need_mask) apply_mask(1, s1);
      const float a1 = half_max(s1);
      // PV(0) + exp(1), and the Vᵀ fragments of half 1
      __builtin_amdgcn_sched_barrier(0);
      pv(0, p0);
      half_exp(s1, p1);
      read_v(1);
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // VALU
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // DS read
      }
      pin(p1[0]);
      pin(p1[1]);
      pin(l_run[0]);
      __builtin_amdgcn_sched_barrier(0);
      if (a1 != 1.f) rescale(a1);
      pv(1, p1);
    }

    if (kvt + 1 < nkv) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  };
  for (int kvt = 0; kvt < nkv; kvt += 2) {
    tile(kvt, std::integral_constant<int, 0>{});
    if (kvt + 1 < nkv) tile(kvt + 1, std::integral_constant<int, 1>{});
  }

  // ---- epilogue: back to the true max, normalise, store
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qrow = qw0 + 32 * qb + l32;
    // a and l are both relative to m_run; the carrier is relative to m_true
    float fix = 1.f;
    if (m_true[qb] != -__builtin_inff() && m_run[qb] != -__builtin_inff())
      fix = __builtin_amdgcn_exp2f((m_run[qb] - m_true[qb]) * c);
    const float l_sum = l_run[qb] + __shfl_xor(l_run[qb], 32, 64);
    const float l_tot = l_sum * fix;
    if (qrow >= Tq) continue;
    const float inv = normalize ? 1.0f / l_sum : fix;
    // fully masked row: 0/0 = NaN for om_apply (normalize 1), 0 for sdpa (2)
    const bool empty_row = normalize && l_sum == 0.f;
    const float fill = normalize == 2 ? 0.f : __builtin_nanf("");
    uint16_t* orow = o + (int64_t)qrow * ost;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int d = 32 * db + 8 * rg + 4 * g;
        float x0 = oacc[db][qb][4 * rg + 0] * inv, x1 = oacc[db][qb][4 * rg + 1] * inv;
        float x2 = oacc[db][qb][4 * rg + 2] * inv, x3 = oacc[db][qb][4 * rg + 3] * inv;
        if (empty_row) x0 = x1 = x2 = x3 = fill;
        *reinterpret_cast<u32x2*>(orow + d) = u32x2{pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)};
      }
    }
    if (g == 0) {
      const int64_t mi = (b * H + h) * (int64_t)Tq + qrow;
      if (m_out) m_out[mi] = m_true[qb] * m_unit;  // natural-log units of the scaled score
      if (l_out) l_out[mi] = l_tot;
    }
  }
}

// ------------------------------------------------ 64 queries per wave (D = 128)
// One workgroup = 4 waves over a query tile of 256 queries of one (b, h) (or
// two such tiles in turn), 64 per wave, one wave per SIMD (512 registers: the
// O accumulators, Q and K fragments in AGPRs).
// Every K / Vᵀ fragment a wave reads from LDS feeds two MFMAs, half the LDS
// bytes per MFMA of the 32-query kernel above.  The tile loop is the inline
// asm of attn_q64_loop.inc (generated by gen_attn_q64.py, which documents
// its registers, the software pipeline of the softmax across tiles, the LDS
// ring and the waits); this C++ computes its addresses and bounds and does
// the epilogue.  Keys come in whole 64-key tiles (Tk a multiple of 64, no
// key mask): causal and unmasked leaves only.
constexpr int QT64 = 256;                // queries per query tile (a workgroup takes one or two)
constexpr int LDS64 = 128 * 1024;        // three 32 KB tile stages; O staged through it after the loop

// Workgroups that take two query tiles of one (b, h), tiles p and nqt - 1 - p
// (nqt even): every causal pair then holds the same number of key tiles, so
// the grid stays balanced without a longest-first order, and a CU starts half
// as many workgroups (each start costs a dispatch gap of its own, and the
// second tile's loads start while the first tile's stores drain).  Each XCD
// owns a contiguous range of heads and takes them in order, pairs of a head
// together.
__device__ __forceinline__ void pair_of_block(int npair, int& bh, int& p) {
  const int nblk = gridDim.x, nbh = nblk / npair;
  int w = blockIdx.x;
  if ((nblk & 7) == 0 && (nbh & 7) == 0) {
    const int hx = nbh >> 3, kk = w >> 3;
    bh = (w & 7) * hx + kk / npair;
    p = kk - (kk / npair) * npair;
    return;
  }
  if ((nblk & 7) == 0) w = (w & 7) * (nblk >> 3) + (w >> 3);
  bh = w / npair;
  p = w - bh * npair;
}

template <int MASK>
__global__ __launch_bounds__(NT, 1) void attn_q64_kernel(
    const uint16_t* __restrict__ q, int64_t qsb, int64_t qsh, int64_t qst,
    const uint16_t* __restrict__ k, int64_t ksb, int64_t ksh, int64_t kst,
    const uint16_t* __restrict__ v, int64_t vsb, int64_t vsh, int64_t vst,
    uint16_t* __restrict__ o, int64_t osb, int64_t osh, int64_t ost, float* __restrict__ m_out,
    float* __restrict__ l_out, int H, int Tq, int Tk, float scale, int64_t causal_off, int normalize,
    int paired) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int nqt = (Tq + QT64 - 1) / QT64;
  // the workgroup's query tiles: the short one of a causal pair first
  int bh, qt_first, ntile;
  if (paired) {
    int p;
    pair_of_block(nqt >> 1, bh, p);
    qt_first = p;
    ntile = 2;
  } else {
    int qi;
    tile_of_block(nqt, bh, qi);
    qt_first = (MASK == CATOPT_MASK_CAUSAL) ? (nqt - 1 - qi) : qi;
    ntile = 1;
  }
  const int64_t b = bh / H, h = bh - (int64_t)(bh / H) * H;
  q += b * qsb + h * qsh;
  k += b * ksb + h * ksh;
  v += b * vsb + h * vsh;
  o += b * osb + h * osh;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5, G = lane >> 4, jj = lane & 15;
  const float c = scale * 1.4426950408889634f;

  const uint32_t lb = lds_u32(lds);
  const u32x4 krs = make_rsrc(k, (uint32_t)(((int64_t)(Tk - 1) * kst + 128) * 2));
  const u32x4 vrs = make_rsrc(v, (uint32_t)(((int64_t)(Tk - 1) * vst + 128) * 2));
  const uint32_t kstep = __builtin_amdgcn_readfirstlane((uint32_t)(64 * kst * 2));
  const uint32_t vstep = __builtin_amdgcn_readfirstlane((uint32_t)(64 * vst * 2));
  const uint32_t dmab = __builtin_amdgcn_readfirstlane(lb + wave * 1024);
  const float s_c = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, c)));

#pragma unroll 1
  for (int pt = 0; pt < ntile; ++pt) {
    const int qt = pt == 0 ? qt_first : nqt - 1 - qt_first;
    const int q0 = qt * QT64;
    const int qw0 = q0 + wave * 64;  // first query of this wave

    // tiles of the workgroup (nkv), of this wave (wnt: a wave past Tq
    // computes none) and the first one reaching past the wave's first query
    // (mfrom: from there on the causal mask applies)
    int64_t kv_end = Tk, wave_end = Tk, mfrom64 = 0x7fffffff;
    if (MASK == CATOPT_MASK_CAUSAL) {
      const int64_t lim = (int64_t)q0 + QT64 + causal_off;
      kv_end = lim < 0 ? 0 : (lim < Tk ? lim : Tk);
      const int64_t wl_end = (int64_t)qw0 + 64 + causal_off;
      wave_end = wl_end < 0 ? 0 : (wl_end < Tk ? wl_end : Tk);
      const int64_t x = (int64_t)qw0 + causal_off - 63;  // first tile t with 64 t > x
      const int64_t fl = x >= 0 ? x / 64 : -((-x + 63) / 64);
      mfrom64 = fl + 1 < 0 ? 0 : fl + 1;
    }
    const int nkv = (int)((kv_end + 63) / 64);
    const int wnt = qw0 < Tq ? (int)((wave_end + 63) / 64) : 0;
    const int mfrom = (int)(mfrom64 < nkv ? mfrom64 : nkv);
    int64_t l0 = (int64_t)qw0 + causal_off;  // (keys and queries stay below 2^31)
    l0 = l0 < -(1LL << 30) ? -(1LL << 30) : (l0 > (1LL << 30) ? (1LL << 30) : l0);
    const int lim0 = (int)l0 + l32 - 4 * g;
    uint64_t qa[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      int row = qw0 + 32 * qb + l32;
      row = row < Tq ? row : Tq - 1;  // rows past Tq load a valid row; their outputs are dropped
      qa[qb] = reinterpret_cast<uint64_t>(q + (int64_t)row * qst) + 16 * g;
    }
    // LDS fragment addresses of stage 0 (stage 1 adds 32 KB in the immediate,
    // stage 2 reads through the second set, 64 KB further): K rows swizzled as
    // tile_off<128>, Vᵀ by the transposing-read swizzle vtile_off<128>.  They
    // are recomputed per tile from a lane index the compiler cannot hoist, so
    // that only scalars stay live across the asm block (hoisted, they spilled).
    int lt = lane;
    asm volatile("" : "+v"(lt));
    const int l32t = lt & 31, gt = lt >> 5, Gt = lt >> 4, jjt = lt & 15;
    uint32_t ka[8], kah[8], va[4], vah[4], ko[4], vo[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ka[j] = lb + tile_off<128>(l32t, 2 * j + gt);
      kah[j] = ka[j] + 65536;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int key0 = 4 * (Gt >> 1) + (jjt >> 2);
      const int d = 32 * db + 16 * (Gt & 1) + 4 * (jjt & 3);
      va[db] = lb + AttnLds<128>::TILE_BYTES + vtile_off<128>(key0, d >> 3) + (d & 7) * 2;
      vah[db] = va[db] + 65536;
    }
    // this thread's four 16-byte slots of a K and of a V tile (byte offsets
    // from the tile's first row; the tile's offset goes in soffset)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int s = i * NT + wave * 64 + lt;
      const int row = s / AttnLds<128>::CH, cp = s % AttnLds<128>::CH;
      ko[i] = (uint32_t)(row * (int)kst + (cp ^ (row & 15)) * 8) * 2u;
      vo[i] = (uint32_t)(row * (int)vst + (cp ^ vswz<128>(row)) * 8) * 2u;
    }
    const uint32_t ob = lb + wave * 32768 + lt * 16;
    const int s_nkv = __builtin_amdgcn_readfirstlane(nkv);
    const int s_wnt = __builtin_amdgcn_readfirstlane(wnt);
    const int s_mfrom = __builtin_amdgcn_readfirstlane(mfrom);

    float m_run[2], m_true[2], l_run[2];
    int st_t, st_kv0, st_kso, st_vso, st_tmp, st_fl0, st_fl1;
    asm volatile(ATTN_Q64_ASM
                 : [mr0] "=&v"(m_run[0]), [mr1] "=&v"(m_run[1]), [mt0] "=&v"(m_true[0]),
                   [mt1] "=&v"(m_true[1]), [lr0] "=&v"(l_run[0]), [lr1] "=&v"(l_run[1]),
                   [t] "=&s"(st_t), [kv0] "=&s"(st_kv0), [kso] "=&s"(st_kso), [vso] "=&s"(st_vso),
                   [tmp] "=&s"(st_tmp), [fl0] "=&s"(st_fl0), [fl1] "=&s"(st_fl1)
                 : [nkv] "s"(s_nkv), [wnt] "s"(s_wnt), [mfrom] "s"(s_mfrom), [krs] "s"(krs), [vrs] "s"(vrs),
                   [kstep] "s"(kstep), [vstep] "s"(vstep), [dmab] "s"(dmab), [c] "s"(s_c), [lim0] "v"(lim0),
                   [ka0] "v"(ka[0]), [ka1] "v"(ka[1]), [ka2] "v"(ka[2]), [ka3] "v"(ka[3]), [ka4] "v"(ka[4]),
                   [ka5] "v"(ka[5]), [ka6] "v"(ka[6]), [ka7] "v"(ka[7]), [kah0] "v"(kah[0]), [kah1] "v"(kah[1]),
                   [kah2] "v"(kah[2]), [kah3] "v"(kah[3]), [kah4] "v"(kah[4]), [kah5] "v"(kah[5]),
                   [kah6] "v"(kah[6]), [kah7] "v"(kah[7]), [va0] "v"(va[0]), [va1] "v"(va[1]), [va2] "v"(va[2]),
                   [va3] "v"(va[3]), [vah0] "v"(vah[0]), [vah1] "v"(vah[1]), [vah2] "v"(vah[2]),
                   [vah3] "v"(vah[3]), [ko0] "v"(ko[0]), [ko1] "v"(ko[1]), [ko2] "v"(ko[2]), [ko3] "v"(ko[3]),
                   [vo0] "v"(vo[0]), [vo1] "v"(vo[1]), [vo2] "v"(vo[2]), [vo3] "v"(vo[3]), [qa0] "v"(qa[0]),
                   [qa1] "v"(qa[1]), [ob] "v"(ob)
                 : "memory", "m0", "vcc", "scc", ATTN_Q64_CLOBBERS);

    // ---- epilogue (as attn_fwd_kernel's): O from LDS (all 32 reads in
    // flight at once), back to the true max, normalise; the bf16 rows go back
    // into the wave's own LDS region (row r at 256 r, its 16-byte chunk c in
    // slot c ^ (r % 16), so that neither the scattered writes nor the row
    // reads collide in a bank) and leave as whole 256-byte rows, four rows
    // per store instruction.  A lane holds query row 32 qb + l32, dims
    // 32 db + 8 rg + 4 g .. +3 of (qb, db, rg).
    char* wl = lds + wave * 32768;
    int le = lane;  // opaque again: the epilogue's addresses stay in the loop too
    asm volatile("" : "+v"(le));
    const int l32e = le & 31, ge = le >> 5;
    f32x4 ox[2][4][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg)
          ox[qb][db][rg] = *reinterpret_cast<const f32x4*>(wl + le * 16 + ((qb * 4 + db) * 4 + rg) * 1024);
    u32x2 ov[2][4][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int qrow = qw0 + 32 * qb + l32e;
      float fix = 1.f;
      if (m_true[qb] != -__builtin_inff() && m_run[qb] != -__builtin_inff())
        fix = __builtin_amdgcn_exp2f((m_run[qb] - m_true[qb]) * c);
      const float l_sum = l_run[qb] + __shfl_xor(l_run[qb], 32, 64);
      const float l_tot = l_sum * fix;
      const float inv = normalize ? 1.0f / l_sum : fix;
      const bool empty_row = normalize && l_sum == 0.f;
      const float fill = normalize == 2 ? 0.f : __builtin_nanf("");
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const f32x4 x = ox[qb][db][rg];
          float x0 = x[0] * inv, x1 = x[1] * inv, x2 = x[2] * inv, x3 = x[3] * inv;
          if (empty_row) x0 = x1 = x2 = x3 = fill;
          ov[qb][db][rg] = u32x2{pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)};
        }
      }
      if (ge == 0 && qrow < Tq) {
        const int64_t mi = (b * H + h) * (int64_t)Tq + qrow;
        if (m_out) m_out[mi] = m_true[qb] * scale;  // natural-log units of the scaled score
        if (l_out) l_out[mi] = l_tot;
      }
    }
    // every lane's fp32 reads have returned before any bf16 row overwrites them
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int r = 32 * qb + l32e, ch = 4 * db + rg;
          *reinterpret_cast<u32x2*>(wl + r * 256 + ((ch ^ (r & 15)) << 4) + 8 * ge) = ov[qb][db][rg];
        }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int ch = le & 15;
    u32x4 rows[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = 4 * j + (le >> 4);
      rows[j] = *reinterpret_cast<const u32x4*>(wl + r * 256 + ((ch ^ (r & 15)) << 4));
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = 4 * j + (le >> 4);
      if (qw0 + r < Tq) *reinterpret_cast<u32x4*>(o + (int64_t)(qw0 + r) * ost + 8 * ch) = rows[j];
    }
    // the next tile's loads go into LDS that every wave has read out
    if (pt + 1 < ntile) __syncthreads();
  }
}

template <int MASK>
int32_t attn_q64_launch(const uint16_t* q, const int64_t* qs, const uint16_t* k, const int64_t* ks,
                        const uint16_t* v, const int64_t* vs, uint16_t* o, const int64_t* os, float* m_out,
                        float* l_out, int64_t B, int64_t H, int64_t Tq, int64_t Tk, float scale,
                        int64_t causal_off, int normalize, hipStream_t s) {
  static bool attr_done = false;
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_q64_kernel<MASK>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS64);
    if (e != hipSuccess) return set_hip_error(e);
    attr_done = true;
  }
  const int64_t nqt = (Tq + QT64 - 1) / QT64;
  // an even number of query tiles goes two to a workgroup
  const int paired = nqt % 2 == 0 ? 1 : 0;
  const int64_t nblk = (paired ? nqt / 2 : nqt) * H * B;
  if (nblk > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;
  attn_q64_kernel<MASK><<<dim3((uint32_t)nblk), dim3(NT), LDS64, s>>>(
      q, qs[0], qs[1], qs[2], k, ks[0], ks[1], ks[2], v, vs[0], vs[1], vs[2], o, os[0], os[1], os[2], m_out,
      l_out, (int)H, (int)Tq, (int)Tk, scale, causal_off, normalize, paired);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

// The 64-query kernel takes bf16, D = 128, no mask or causal, whole 64-key
// tiles, and K / V heads whose buffer ranges fit 31 bits.
bool q64_fits(int64_t d, int32_t mode, int64_t Tk, const int64_t* ks, const int64_t* vs) {
  if (d != 128 || (mode != CATOPT_MASK_NONE && mode != CATOPT_MASK_CAUSAL)) return false;
  if (Tk <= 0 || Tk % 64 != 0) return false;
  return ((Tk - 1) * ks[2] + 128) * 2 < 0x7fffffffLL && ((Tk - 1) * vs[2] + 128) * 2 < 0x7fffffffLL;
}

template <int D, int MASK>
int32_t attn_launch(const uint16_t* q, const int64_t* qs, const uint16_t* k, const int64_t* ks,
                    const uint16_t* v, const int64_t* vs, uint16_t* o, const int64_t* os,
                    float* m_out, float* l_out, int64_t B, int64_t H, int64_t Tq, int64_t Tk,
                    float scale, int64_t causal_off, const void* mask, int64_t mask_ld,
                    int normalize, hipStream_t s) {
  static bool attr_done = false;
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_fwd_kernel<D, MASK>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, AttnLds<D>::BYTES);
    if (e != hipSuccess) return set_hip_error(e);
    attr_done = true;
  }
  const int64_t nqt = (Tq + QT - 1) / QT;
  const int64_t nblk = nqt * H * B;
  if (nblk > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;
  attn_fwd_kernel<D, MASK><<<dim3((uint32_t)nblk), dim3(NT), AttnLds<D>::BYTES, s>>>(
      q, qs[0], qs[1], qs[2], k, ks[0], ks[1], ks[2], v, vs[0], vs[1], vs[2], o, os[0], os[1],
      os[2], m_out, l_out, (int)H, (int)Tq, (int)Tk, scale, causal_off, mask, mask_ld, normalize);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

template <int D>
int32_t attn_dispatch_mask(int32_t mode, const uint16_t* q, const int64_t* qs, const uint16_t* k,
                           const int64_t* ks, const uint16_t* v, const int64_t* vs, uint16_t* o,
                           const int64_t* os, float* m_out, float* l_out, int64_t B, int64_t H,
                           int64_t Tq, int64_t Tk, float scale, int64_t causal_off,
                           const void* mask, int64_t mask_ld, int normalize, hipStream_t s) {
  switch (mode) {
    case CATOPT_MASK_NONE:
      return attn_launch<D, CATOPT_MASK_NONE>(q, qs, k, ks, v, vs, o, os, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask, mask_ld, normalize, s);
    case CATOPT_MASK_CAUSAL:
      return attn_launch<D, CATOPT_MASK_CAUSAL>(q, qs, k, ks, v, vs, o, os, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask, mask_ld, normalize, s);
    case CATOPT_MASK_BOOL:
      return attn_launch<D, CATOPT_MASK_BOOL>(q, qs, k, ks, v, vs, o, os, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask, mask_ld, normalize, s);
    case CATOPT_MASK_BIAS:
      return attn_launch<D, CATOPT_MASK_BIAS>(q, qs, k, ks, v, vs, o, os, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask, mask_ld, normalize, s);
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
                                       int64_t causal_off, const void* mask, int64_t mask_ld,
                                       int32_t normalize, void* o, const int64_t* o_strides,
                                       float* m_out, float* l_out, void* stream) {
  if (B < 0 || H < 0 || Tq < 0 || Tk < 0) return CATOPT_E_INVAL;
  if (mask_mode < CATOPT_MASK_NONE || mask_mode > CATOPT_MASK_BIAS) return CATOPT_E_INVAL;
  if (normalize < 0 || normalize > 2) return CATOPT_E_INVAL;
  if (dtype != CATOPT_BF16) return CATOPT_E_UNSUPPORTED;
  if (d != dv || (d != 128 && d != 64)) return CATOPT_E_UNSUPPORTED;
  if (!(scale > 0.f) || !__builtin_isfinite(scale)) return CATOPT_E_UNSUPPORTED;
  if (B == 0 || H == 0 || Tq == 0) return CATOPT_OK;
  // no keys: k and v may be empty (null) buffers; every row is the empty carrier
  if (!q || !o || (Tk > 0 && (!k || !v))) return CATOPT_E_INVAL;
  if (!strides_ok(q_strides) || !strides_ok(k_strides) || !strides_ok(v_strides) ||
      !strides_ok(o_strides))
    return CATOPT_E_INVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return CATOPT_E_INVAL;
  if ((mask_mode == CATOPT_MASK_BOOL || mask_mode == CATOPT_MASK_BIAS) && (!mask || mask_ld < Tk))
    return CATOPT_E_INVAL;
  if (mask_mode == CATOPT_MASK_BIAS && (reinterpret_cast<uintptr_t>(mask) & 3)) return CATOPT_E_INVAL;
  if (Tq > 0x7fffffffLL || Tk > 0x7fffffffLL || H > 65535 || B > 65535) return CATOPT_E_UNSUPPORTED;
  // per-thread tile offsets are 32-bit: 64 rows of either stride must fit
  if ((k_strides[2] + 1) * 64 + d >= 0x7fffffffLL || (v_strides[2] + 1) * 64 + d >= 0x7fffffffLL)
    return CATOPT_E_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto qp = static_cast<const uint16_t*>(q);
  auto kp = static_cast<const uint16_t*>(k);
  auto vp = static_cast<const uint16_t*>(v);
  auto op = static_cast<uint16_t*>(o);
  if (q64_fits(d, mask_mode, Tk, k_strides, v_strides)) {
    if (mask_mode == CATOPT_MASK_CAUSAL)
      return attn_q64_launch<CATOPT_MASK_CAUSAL>(qp, q_strides, kp, k_strides, vp, v_strides, op, o_strides,
                                                 m_out, l_out, B, H, Tq, Tk, scale, causal_off, normalize, s);
    return attn_q64_launch<CATOPT_MASK_NONE>(qp, q_strides, kp, k_strides, vp, v_strides, op, o_strides, m_out,
                                             l_out, B, H, Tq, Tk, scale, causal_off, normalize, s);
  }
  if (d == 128)
    return attn_dispatch_mask<128>(mask_mode, qp, q_strides, kp, k_strides, vp, v_strides, op,
                                   o_strides, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask,
                                   mask_ld, normalize, s);
  return attn_dispatch_mask<64>(mask_mode, qp, q_strides, kp, k_strides, vp, v_strides, op,
                                o_strides, m_out, l_out, B, H, Tq, Tk, scale, causal_off, mask,
                                mask_ld, normalize, s);
}
