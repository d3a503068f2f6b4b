// Chunked decayed retention on fp32 operands (gfx950 fp32 MFMA,
// v_mfma_f32_32x32x2_f32):
//
//   o[t] = scale · Σ_{s ≤ t} γ^(t−s) (q[t]·k[s]) v[s]
//
// in chunks of C = 64 steps: for chunk n with carried state S (d × dv),
//   o_n = scale · ( (q_n k_nᵀ ⊙ D) v_n + diag(γ^a) q_n S ),   D[a, b] = γ^(a−b) (a ≥ b)
//   S  ← γ^C S + k_nᵀ diag(γ^(C−b)) v_n
// which is the bf16 kernel's algebra with every operand, product and the
// state in fp32 (no rounding to bf16 anywhere).
//
// Work split.  A workgroup owns one head and a slice of 32 value columns and
// runs every chunk in order.  Wave w owns q/k columns [32w, 32w + 32): its
// share of the score q kᵀ, of the inter-chunk term q S and of the state
// update only ever touches those columns, and all three are linear in them,
// so each wave produces a partial output of the chunk's 64 x 32 block; the
// four partials are summed through LDS once per chunk (double-buffered, one
// barrier per chunk).  The state tile S[32w.., slice] stays in registers.
//
// Operand layouts (32x32x2 f32 MFMA: lane l gives A row l%32 and B column
// l%32 at k index l/32; the accumulator of lane l holds column l%32, rows
// acc_row(r, l/32) in register r).  The k index of a product is a summation
// order, so k-step t with half-wave g can take any inner index as long as A
// and B agree; every product here takes inner index acc_row(t, g) (plus the
// tile base), which lets accumulators feed the next product directly:
//   * the state accumulator S[dd, c] (lane: column c, register t: row dd)
//     is the B operand of the inter term O = Q S;
//   * the score accumulator Pᵀ[j, i] (lane: query i, register t: key j) is
//     the A operand of O += P V;
//   * q and k are loaded so that register t of lane (row, g) holds column
//     acc_row(t, g) of the wave's 32 columns (four 16-byte loads per tile).
// v and the key columns of the state update (kᵀ) are read with lanes along
// a row (128-byte coalesced words).  Loads go through buffer resources over
// the head's rows: rows past T read zeros; columns past d are given an
// out-of-range offset and read zeros too.
#include "common.hpp"

namespace catopt {
namespace {

constexpr int kC = 64;          // chunk length (steps)
constexpr int kNT = 256;        // 4 waves
constexpr int kSlice = 32;      // value columns per workgroup
constexpr uint32_t kOOB = 0x80000000u;  // a buffer offset past every range: loads 0

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4 ld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

__device__ __forceinline__ float ld1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}

// Byte offset of column `col` in a row, or kOOB past the row's width d.  It
// is added to row offsets below 2^31, so a past-the-width column stays out of
// range; computed once per lane (and kept opaque) so that no load carries a
// select the compiler could split into branches around the load.
__device__ __forceinline__ uint32_t col_bytes(int col, int d) {
  uint32_t c = col < d ? (uint32_t)col * 4u : kOOB;
  asm volatile("" : "+v"(c));
  return c;
}

// Row-tile operand of q or k: reg[4u + e] = X[row0 + l32][dd0 + 8u + 4g + e]
// with vrow[u] = l32·d·4 + col_bytes(dd0 + 8u + 4g) and soff = row0·d·4.
__device__ __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t r, const uint32_t (&vrow)[4], uint32_t soff,
                                          float (&reg)[16]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float4 x = ld4(r, vrow[u], soff);
    reg[4 * u + 0] = x.x;
    reg[4 * u + 1] = x.y;
    reg[4 * u + 2] = x.z;
    reg[4 * u + 3] = x.w;
  }
}

// Column operand: reg[t] = X[row0 + acc_row(t, g)][col] with
// vcol = 4g·d·4 + col_bytes(col) and soff = row0·d·4; the rest of the row
// index, 8(t/4) + t%4, goes into the scalar offset.
__device__ __forceinline__ void load_cols(__amdgpu_buffer_rsrc_t r, uint32_t vcol, uint32_t soff, int d,
                                          float (&reg)[16]) {
#pragma unroll
  for (int t = 0; t < 16; ++t) reg[t] = ld1(r, vcol, soff + (uint32_t)((8 * (t >> 2) + (t & 3)) * d * 4));
}

__global__ __launch_bounds__(kNT) void retention_f32(const float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, const float* __restrict__ gamma,
                                                     float scale, float* __restrict__ o, int H, int T, int d,
                                                     int nslice, int remap_rows) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [2][4][64][32] partial outputs
  // XCD-aware order: the hardware deals workgroups to the 8 XCDs round-robin;
  // remapping keeps consecutive logical ids (a head's slices, which read the
  // same q and k) on one XCD's L2
  int bid = blockIdx.x;
  if (remap_rows > 0) bid = (bid & 7) * remap_rows + (bid >> 3);
  const int slice = bid % nslice;
  const int64_t bh = bid / nslice;
  const int h = (int)(bh % H);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int dd0 = 32 * w;            // this wave's q/k columns
  const int c0 = kSlice * slice;     // this workgroup's value columns
  const int nact = (d + 31) / 32;    // waves holding q/k columns
  const bool active = dd0 < d;
  const int64_t base = bh * (int64_t)T * d;
  const int bytes = T * d * 4;
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)(q + base), (short)0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)(k + base), (short)0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)(v + base), (short)0, bytes, 0x00020000);
  float* oh = o + base;

  // decay factors of this lane, fixed over the chunks (exp2 domain)
  const float gam = gamma[h];
  const float lg = log2f(fabsf(gam));
  const bool neg = gam < 0.f;
  float rowf[2][16], diagf[16], offf[16], wv[2][16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int ar = acc_row(r, g);
    rowf[0][r] = pow_k(lg, neg, ar);                             // γ^a, a = row in chunk
    rowf[1][r] = pow_k(lg, neg, 32 + ar);
    diagf[r] = ar <= l32 ? pow_k(lg, neg, l32 - ar) : 0.f;        // D on diagonal tiles
    offf[r] = pow_k(lg, neg, 32 + l32 - ar);                      // D on the lower tile
    wv[0][r] = pow_k(lg, neg, kC - ar);                           // γ^(C − b)
    wv[1][r] = pow_k(lg, neg, kC - 32 - ar);
  }
  const float gC = pow_k(lg, neg, kC);

  // per-lane parts of the load offsets (bytes); row bases go to soffset
  uint32_t vrow[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) vrow[u] = (uint32_t)(l32 * d * 4) + col_bytes(dd0 + 8 * u + 4 * g, d);
  const uint32_t vcol_v = (uint32_t)(4 * g * d * 4) + col_bytes(c0 + l32, d);
  const uint32_t vcol_k = (uint32_t)(4 * g * d * 4) + col_bytes(dd0 + l32, d);
  const uint32_t tile_b = 32u * (uint32_t)d * 4u;  // bytes of 32 rows

  f32x16 sacc = {};  // S[dd0 + acc_row(r, g)][c0 + l32]
  const int nch = (T + kC - 1) / kC;
  float qr[2][16], kr[2][16];
  if (active) {
    load_rows(rq, vrow, 0, qr[0]);
    load_rows(rq, vrow, tile_b, qr[1]);
    load_rows(rk, vrow, 0, kr[0]);
    load_rows(rk, vrow, tile_b, kr[1]);
  }
  for (int n = 0; n < nch; ++n) {
    const int t0 = n * kC;
    const uint32_t sb = (uint32_t)t0 * (uint32_t)d * 4u;  // the chunk's first row
    float* buf = red + (n & 1) * (4 * kC * kSlice);
    if (active) {
      float vr[2][16], kc[2][16];
      load_cols(rv, vcol_v, sb, d, vr[0]);
      load_cols(rv, vcol_v, sb + tile_b, d, vr[1]);
      load_cols(rk, vcol_k, sb, d, kc[0]);
      load_cols(rk, vcol_k, sb + tile_b, d, kc[1]);

      // inter-chunk term, then the per-row decay γ^a
      f32x16 oacc[2] = {{}, {}};
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        oacc[0] = mfma_f32(qr[0][t], sacc[t], oacc[0]);
        oacc[1] = mfma_f32(qr[1][t], sacc[t], oacc[1]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        oacc[0][r] *= rowf[0][r];
        oacc[1][r] *= rowf[1][r];
      }
      // scores Pᵀ[j, i] over this wave's columns: tiles (jt, it) = (0,0), (0,1), (1,1)
      f32x16 p00 = {}, p01 = {}, p11 = {};
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        p00 = mfma_f32(kr[0][t], qr[0][t], p00);
        p01 = mfma_f32(kr[0][t], qr[1][t], p01);
        p11 = mfma_f32(kr[1][t], qr[1][t], p11);
      }
      // the next chunk's q and k rows (their registers are free from here)
      if (n + 1 < nch) {
        const uint32_t nb = sb + 2u * tile_b;
        load_rows(rq, vrow, nb, qr[0]);
        load_rows(rq, vrow, nb + tile_b, qr[1]);
        load_rows(rk, vrow, nb, kr[0]);
        load_rows(rk, vrow, nb + tile_b, kr[1]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p00[r] *= diagf[r];
        p11[r] *= diagf[r];
        p01[r] *= offf[r];
      }
      // intra-chunk term O += P V (query tile 0 sees key tile 0, tile 1 both)
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        oacc[0] = mfma_f32(p00[t], vr[0][t], oacc[0]);
        oacc[1] = mfma_f32(p01[t], vr[0][t], oacc[1]);
        oacc[1] = mfma_f32(p11[t], vr[1][t], oacc[1]);
      }
      // state update S ← γ^C S + kᵀ diag(γ^(C−b)) v over this wave's rows
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] *= gC;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        sacc = mfma_f32(kc[0][t], wv[0][t] * vr[0][t], sacc);
        sacc = mfma_f32(kc[1][t], wv[1][t] * vr[1][t], sacc);
      }
      float* mine = buf + w * (kC * kSlice);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        mine[acc_row(r, g) * kSlice + l32] = oacc[0][r];
        mine[(32 + acc_row(r, g)) * kSlice + l32] = oacc[1][r];
      }
    }
    __syncthreads();
    // wave w sums and stores rows 8w .. 8w + 7 of each 32-row half
    const int col = c0 + l32;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int i = 32 * it + 8 * w + 4 * g + e;
        float s = 0.f;
#pragma unroll
        for (int x = 0; x < 4; ++x) {  // partials of waves past nact were not written: selected out
          const float px = buf[x * (kC * kSlice) + i * kSlice + l32];
          s += x < nact ? px : 0.f;
        }
        const int row = t0 + i;
        if (row < T && col < d) oh[(int64_t)row * d + col] = scale * s;
      }
    }
  }
}

}  // namespace

int32_t retention_f32_launch(int64_t B, int64_t H, int64_t T, int64_t d, const float* q, const float* k,
                             const float* v, const float* gamma, float scale, float* o, hipStream_t s) {
  if (d < 1 || d > 128 || d % 4) return CATOPT_E_UNSUPPORTED;
  if (T * d * 4 + (int64_t)kC * d * 4 > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;  // 32-bit buffer offsets
  const int nslice = (int)((d + kSlice - 1) / kSlice);
  const int64_t grid = B * H * nslice;
  if (grid > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;
  const int remap_rows = grid % 8 == 0 ? (int)(grid / 8) : 0;
  const size_t lds = 2 * 4 * kC * kSlice * sizeof(float);
  retention_f32<<<dim3((uint32_t)grid), dim3(kNT), lds, s>>>(q, k, v, gamma, scale, o, (int)H, (int)T, (int)d,
                                                             nslice, remap_rows);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

}  // namespace catopt
