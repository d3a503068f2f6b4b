// Chunked decayed retention (RetNet) for gfx950, bf16 in / fp32 state.
//
//   o[t] = scale * sum_{s <= t} γ^(t-s) (q[t]·k[s]) v[s]
//
// evaluated chunk-wise with chunk length C = 64 and head dim 128.  Chunk i
// (rows t = iC + q) takes its diagonal block with decay(γ, C) and every
// strict-lower block through the carried state
//   S_i = sum_{j<i} sum_c γ^((i-j)C - c) k_jc ⊗ v_jc,   S_{i+1} = γ^C S_i + sum_c γ^(C-c) k_ic ⊗ v_ic,
// so that  o_i = scale * ( (q_i k_iᵀ ⊙ D) v_i + diag(γ^q) q_i S_i ),  D[q][c] = γ^(q-c) (c <= q):
// the K-way block decomposition's algebra, with its rank-1 decay_vec factors
// γ^(q + (i-j)C) · γ^(-c) folded into the state.
//
// Single pass.  One workgroup per (b, h, 32-column slice of v): the state
// slice S[:, slice] (128 x 32 fp32) stays in registers while the workgroup
// walks its head's chunks in order, so q, k, v and o each cross HBM once.
// The four slices of a head are dealt to one XCD (workgroups go round robin
// over the 8 XCDs), so the q and k chunks all four read come from its L2.
//
// Per chunk, 4 waves, 32x32x16 bf16 MFMA with fp32 accumulation, all
// products computed transposed (output column = query):
//   wave (kb, qb) = (w >> 1, w & 1), keys 32kb.., queries 32qb..:
//     X  = Sᵀ[:, dk half kb] Qᵀ          A = S fragments (LDS, bf16), B = q rows
//     X *= scale γ^q                      (per lane: the lane's column is q)
//     sᵀ = K Qᵀ  (kb <= qb only)          A = k rows, B = q rows
//     X += Vᵀ (sᵀ ⊙ scale Dᵀ)             A = v via the transposing LDS read,
//                                         B = P straight from the sᵀ accumulator
//   wave w owns state rows dk = 32w..32w+31:
//     S = γ^C S + Kᵀ (γ^(C-c) V)          A = k via the transposing LDS read,
//                                         B = v likewise, each lane decaying
//                                         its own elements in registers
//   o[q] = X(0, qb) + X(1, qb), the pair meeting in LDS.
// One barrier per chunk: the state update reads no shared decayed copy of v,
// the S fragments and the pair exchange alternate between two LDS buffers by
// chunk parity, and waves (0, qb) store chunk i's output at the start of
// chunk i + 1, once the partner's half is in place.  Within a wave the
// chains X, sᵀ and S are independent, and their MFMAs are interleaved.
// An MFMA's k index is only a summation order: products over keys take their
// keys in the sᵀ accumulator's row order 8(r/4) + 4g + r%4 (so P feeds an
// MFMA without a shuffle), products over dk take dims in natural order, and
// the owner waves re-lay their state rows into natural order in LDS.
//
// Tiles reach LDS by direct global->LDS loads through a ring of NSTAGE
// stages: chunk i + NSTAGE - 1's loads are issued before chunk i's arithmetic,
// which keeps several chunks of loads in flight per workgroup (one workgroup
// per CU leaves nothing else to hide the memory latency behind).
#include <type_traits>

#include "common.hpp"

namespace catopt {
namespace {

constexpr int NT = 256;
constexpr int CH = 64;    // chunk length
constexpr int HD = 128;   // head dim (dk = dv)
constexpr int SL = 32;    // v columns per workgroup
constexpr int NSL = HD / SL;

typedef __attribute__((ext_vector_type(4))) short s16x4;

// LDS layout (bytes).  Per stage: k and q tiles [64][128] bf16 whose 16-byte
// chunks are XOR-swizzled by kq_swz(row), then the v slice [64][32] bf16.
constexpr int KQ_BYTES = CH * HD * 2;             // 16 KB
constexpr int V_BYTES = CH * SL * 2;              // 4 KB
constexpr int STAGE = 2 * KQ_BYTES + V_BYTES;
#ifndef CATOPT_RET_STAGES
#define CATOPT_RET_STAGES 3
#endif
constexpr int NSTAGE = CATOPT_RET_STAGES;
constexpr int SF_BYTES = 4 * 2 * 64 * 16;          // S fragments [4 waves][2][64 lanes] x 16 B
constexpr int X_BYTES = 2 * 4 * 64 * 16;           // pair exchange [2 qb][4][64 lanes] x 16 B
constexpr int OFF_SF = NSTAGE * STAGE;             // two S fragment buffers (chunk parity)
constexpr int OFF_X = OFF_SF + 2 * SF_BYTES;       // two exchange buffers (chunk parity)
constexpr int LDS_BYTES = OFF_X + 2 * X_BYTES;
static_assert(NSTAGE >= 2 && LDS_BYTES <= 160 * 1024, "LDS ring does not fit");
constexpr int LOADS_PER_CHUNK = 9;  // global->LDS instructions per thread per chunk
constexpr int OUT_STORES = 4;       // global stores of one chunk's output per thread (waves kb = 0)

// s_waitcnt: vmcnt <= n, lgkmcnt = 0, expcnt not waited on (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(n >= 0 && n < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | ((n >> 4) << 14));
}

// The 16-byte chunk index of a k / q row is XOR-ed with a bijection of the
// row's position among 16 consecutive rows (low two bits to bits 2-3, bits
// 2-3 to bits 0-1).  A plain row read (16 consecutive rows, one chunk) hits
// 16 distinct chunk slots; a transposing read of k (4 consecutive keys x 4
// adjacent chunks per 32 lanes, rows a whole bank window apart) does too,
// where XOR-ing with (row & 15) folded those 16 pieces onto 4 slots.
__device__ __forceinline__ int kq_swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }
__device__ __forceinline__ int kq_off(int row, int chunk) {  // byte offset in a k / q tile
  return row * (HD * 2) + ((chunk ^ kq_swz(row)) << 4);
}

// Transposing LDS read (ds_read_b64_tr_b16).  Within each 16-lane group, when
// lane j points at row (base + j/4), columns c0 + 4(j%4) .. +3, lane i gets
// column c0 + i of rows base .. base+3.
__device__ __forceinline__ s16x4 ds_read_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
}

__device__ __forceinline__ bf16x8 cat8(s16x4 lo, s16x4 hi) {
  const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
  return __builtin_bit_cast(bf16x8, u32x4{a[0], a[1], b[0], b[1]});
}

__global__ __launch_bounds__(NT, 1) void retention_scan(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ gamma, int H, int64_t T, float scale, uint16_t* __restrict__ o) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  // work item (b*h, slice), the four slices of a head on one XCD
  const int nblk = gridDim.x;
  int wid = blockIdx.x;
  if ((nblk & 7) == 0) wid = (wid & 7) * (nblk >> 3) + (wid >> 3);
  const int64_t bh = wid / NSL;
  const int sl = wid % NSL;
  const int64_t base = bh * T * HD;
  q += base;
  k += base;
  v += base;
  o += base;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int G = lane >> 4, jj = lane & 15;  // 16-lane group, lane within it
  const int kb = wave >> 1, qb = wave & 1;
  const float lg = __log2f(gamma[bh % H]);
  const float gC = __builtin_amdgcn_exp2f((float)CH * lg);
  const int nchunks = (int)(T / CH);
  const int qrow = 32 * qb + l32;  // this lane's query: sᵀ column and output column
  // output scale folded into the per-query and per-entry decay factors
  const float gq = scale * __builtin_amdgcn_exp2f((float)qrow * lg);

  // scale * decay of this lane's sᵀ entries (key 32kb + acc_row(r, g), query qrow)
  float dec[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = 32 * kb + acc_row(r, g);
    dec[r] = key <= qrow ? scale * __builtin_amdgcn_exp2f((float)(qrow - key) * lg) : 0.f;
  }

  // load slots: k and q 4 x 16 B each, v one 16-byte slot
  int kq_goff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = i * NT + wave * 64 + lane;
    const int row = s >> 4, cp = s & 15;
    kq_goff[i] = row * HD + ((cp ^ kq_swz(row)) << 3);
  }
  const int v_goff = (tid >> 2) * HD + sl * SL + (tid & 3) * 8;
  const uint32_t lds_base = lds_u32(lds);

  auto issue = [&](int ci, int stage) {
    const uint32_t sb = lds_base + stage * STAGE + wave * 1024;
    const int64_t t0 = (int64_t)ci * CH * HD;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dma16(k + t0 + kq_goff[i], sb + i * NT * 16);
      dma16(q + t0 + kq_goff[i], sb + KQ_BYTES + i * NT * 16);
    }
    dma16(v + t0 + v_goff, sb + 2 * KQ_BYTES);
  };

  // transposed k rows dk = 32w + 16(G&1) + 4(jj&3) .. for the state update,
  // and transposed v rows dv = 16(G&1) + 4(jj&3) .. (byte offset dvb), both
  // at keys 16u + 4(G>>1) + (0..3, +8)
  const int dk_t = 32 * wave + 16 * (G & 1) + 4 * (jj & 3);
  const int dvb = (16 * (G & 1) + 4 * (jj & 3)) * 2;
  // γ^(C - key) of this lane's transposed-v elements for u = 3 (keys
  // 48 + 4(G>>1) + e, e = 0..3, 8..11); the factors of block u are those of
  // block u + 1 times γ^16, so every exponent stays >= 0
  float vf3[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = 48 + 4 * (G >> 1) + (e < 4 ? e : e + 4);
    vf3[e] = __builtin_amdgcn_exp2f((float)(CH - key) * lg);
  }
  const float g16 = __builtin_amdgcn_exp2f(16.f * lg);

  f32x16 S;  // state rows dk = 32 * wave + acc_row(r, g), column dv = l32 of the slice
#pragma unroll
  for (int r = 0; r < 16; ++r) S[r] = 0.f;
  // S fragments in LDS (two buffers, chunk parity), natural dk order: entry
  // (w, r4, dv) holds bf16 S[32w + 8 r4 + (0..7)][dv]; the owner lane (dv, g)
  // writes its half S[32w + 8 r4 + 4g + (0..3)] = its accumulator registers
  // 4 r4 .. 4 r4 + 3.
  const int sf_own = OFF_SF + (wave * 128 + l32) * 16 + g * 8;  // + par * SF_BYTES + r4 * 512
  const int xch = OFF_X + qb * 4096 + lane * 16;                // + par * X_BYTES + r4 * 1024
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) *reinterpret_cast<u32x2*>(lds + sf_own + r4 * 512) = u32x2{0, 0};
  f32x16 Xo;  // waves kb = 0: their X of the previous chunk, stored once the partner's arrives
#pragma unroll
  for (int r = 0; r < 16; ++r) Xo[r] = 0.f;

  // Prologue: chunks 0 .. NSTAGE-2 in flight.  Every thread issues exactly
  // LOADS_PER_CHUNK loads per chunk slot (a slot past the end re-reads the
  // last chunk into its unused stage), so "all but the newest
  // (NSTAGE-2) groups complete" is one fixed vmcnt.
#pragma unroll
  for (int p = 0; p < NSTAGE - 1; ++p) issue(min(p, nchunks - 1), p);
  wait_vm_lgkm0<LOADS_PER_CHUNK * (NSTAGE - 2)>();
  __syncthreads();

  // o rows of chunk cj for waves kb = 0: own X plus the partner's, read from
  // the exchange buffer of cj's parity
  auto store_out = [&](int cj, const f32x4* y) {
    uint16_t* orow = o + ((int64_t)cj * CH + qrow) * HD + sl * SL + 4 * g;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      *reinterpret_cast<u32x2*>(orow + 8 * r4) =
          u32x2{pack_bf16x2(Xo[4 * r4] + y[r4][0], Xo[4 * r4 + 1] + y[r4][1]),
                pack_bf16x2(Xo[4 * r4 + 2] + y[r4][2], Xo[4 * r4 + 3] + y[r4][3])};
  };

  // One chunk, one barrier: the state update needs no decayed copy of v in
  // LDS (each lane decays its own transposed v elements), the S fragments and
  // the pair exchange alternate between two buffers by chunk parity, and the
  // waves kb = 0 finish chunk ci's output at the start of chunk ci + 1.  The
  // three MFMA chains of a chunk (X, sᵀ, S) are independent and
  // interleaved.  Stage and wave role are compile-time constants.
  auto chunk = [&](int ci, auto stage_tag, auto kb_tag, auto diag_tag) {
    constexpr int cur = decltype(stage_tag)::value;
    constexpr int KB = decltype(kb_tag)::value;
    constexpr bool DIAG = decltype(diag_tag)::value;
    {
      constexpr int st = cur == 0 ? NSTAGE - 1 : cur - 1;  // the stage chunk ci - 1 used
      issue(min(ci + NSTAGE - 1, nchunks - 1), st);
    }
    const char* Ks = lds + cur * STAGE;
    const char* Qs = Ks + KQ_BYTES;
    const char* Vs = Qs + KQ_BYTES;
    const int par = ci & 1;

    // ---- batch: S fragments of dk blocks 2KB, 2KB+1 (this parity), q rows,
    // k rows (diagonal block), transposed k and v, the partner's X of ci-1
    bf16x8 sf[4], qf[8], kf[8], kt[4], vr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sf[i] = *reinterpret_cast<const bf16x8*>(
          lds + OFF_SF + par * SF_BYTES + (((2 * KB + (i >> 1)) * 4 + 2 * (i & 1) + g) * 32 + l32) * 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (DIAG || (j >= 4 * KB && j < 4 * KB + 4))
        qf[j] = *reinterpret_cast<const bf16x8*>(Qs + kq_off(qrow, 2 * j + g));
      if (DIAG) kf[j] = *reinterpret_cast<const bf16x8*>(Ks + kq_off(32 * KB + l32, 2 * j + g));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int key0 = 16 * u + 4 * (G >> 1) + (jj >> 2);
      kt[u] = cat8(ds_read_tr(Ks + kq_off(key0, dk_t >> 3) + (dk_t & 7) * 2),
                   ds_read_tr(Ks + kq_off(key0 + 8, dk_t >> 3) + (dk_t & 7) * 2));
      vr[u] = cat8(ds_read_tr(Vs + key0 * (SL * 2) + dvb), ds_read_tr(Vs + (key0 + 8) * (SL * 2) + dvb));
    }
    f32x4 y[4];
    if (KB == 0) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        y[r4] = *reinterpret_cast<const f32x4*>(lds + xch + (1 - par) * X_BYTES + r4 * 1024);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- interleaved MFMA chains: X = q S (dk half KB), sᵀ = K Qᵀ,
    // S = γ^C S + Kᵀ (γ^(C-c) V)
    f32x16 X, sa;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      X[r] = 0.f;
      sa[r] = 0.f;
      S[r] *= gC;
    }
    float vf[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vf[e] = vf3[e];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int u = 3 - t;  // decay factors run from block 3 down
      X = mfma32x32x16(sf[t], qf[4 * KB + t], X);
      if (DIAG) sa = mfma32x32x16(kf[2 * t], qf[2 * t], sa);
      // element e of vr[u] is bf16 half (e & 1) of word e / 2
      const u32x4 w = __builtin_bit_cast(u32x4, vr[u]);
      u32x4 vd;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2)
        vd[e2] = pack_bf16x2(__uint_as_float(w[e2] << 16) * vf[2 * e2],
                             __uint_as_float(w[e2] & 0xffff0000u) * vf[2 * e2 + 1]);
#pragma unroll
      for (int e = 0; e < 8; ++e) vf[e] *= g16;
      S = mfma32x32x16(kt[u], __builtin_bit_cast(bf16x8, vd), S);
      if (DIAG) sa = mfma32x32x16(kf[2 * t + 1], qf[2 * t + 1], sa);
    }
    if (KB == 0 && ci > 0) store_out(ci - 1, y);

    // ---- X *= scale γ^q; the diagonal block's decayed scores times v
#pragma unroll
    for (int r = 0; r < 16; ++r) X[r] *= gq;
    if (DIAG) {
      bf16x8 pf[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) pf[r >> 3][r & 7] = static_cast<__bf16>(sa[r] * dec[r]);
      X = mfma32x32x16(vr[2 * KB], pf[0], X);
      X = mfma32x32x16(vr[2 * KB + 1], pf[1], X);
    }

    // ---- publish: the partner's half of X, and S_{ci+1} for the next chunk
    if (KB == 1) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        *reinterpret_cast<f32x4*>(lds + xch + par * X_BYTES + r4 * 1024) =
            f32x4{X[4 * r4], X[4 * r4 + 1], X[4 * r4 + 2], X[4 * r4 + 3]};
    } else {
      Xo = X;
    }
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      *reinterpret_cast<u32x2*>(lds + sf_own + (1 - par) * SF_BYTES + r4 * 512) =
          u32x2{pack_bf16x2(S[4 * r4], S[4 * r4 + 1]), pack_bf16x2(S[4 * r4 + 2], S[4 * r4 + 3])};
    // vmcnt counts loads and stores in issue order: chunk ci+1's tiles have
    // landed once no more than chunk ci+2's loads (issued at the top of this
    // chunk) and the output stores issued after them remain
    if (KB == 0 && ci > 0)
      wait_vm_lgkm0<LOADS_PER_CHUNK * (NSTAGE - 2) + OUT_STORES>();
    else
      wait_vm_lgkm0<LOADS_PER_CHUNK * (NSTAGE - 2)>();
    __syncthreads();  // next chunk's tiles, S fragments and this chunk's exchange in place
  };
  auto run = [&](auto kb_tag, auto diag_tag) {
    static_assert(NSTAGE == 3, "the chunk loop below runs three stages");
    for (int ci = 0; ci < nchunks; ci += 3) {
      chunk(ci, std::integral_constant<int, 0>{}, kb_tag, diag_tag);
      if (ci + 1 < nchunks) chunk(ci + 1, std::integral_constant<int, 1>{}, kb_tag, diag_tag);
      if (ci + 2 < nchunks) chunk(ci + 2, std::integral_constant<int, 2>{}, kb_tag, diag_tag);
    }
  };
  // wave roles (kb, qb): (0, *) and (1, 1) take a diagonal block, (1, 0) none
  if (kb == 0)
    run(std::integral_constant<int, 0>{}, std::true_type{});
  else if (qb == 1)
    run(std::integral_constant<int, 1>{}, std::true_type{});
  else
    run(std::integral_constant<int, 1>{}, std::false_type{});
  // the last chunk's output: its exchange is in place after the final barrier
  if (kb == 0) {
    f32x4 y[4];
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      y[r4] = *reinterpret_cast<const f32x4*>(lds + xch + ((nchunks - 1) & 1) * X_BYTES + r4 * 1024);
    store_out(nchunks - 1, y);
  }
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int64_t catopt_hip_retention_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t d,
                                                        int64_t chunk) {
  if (B < 0 || H < 0 || T < 0 || d != HD || chunk != CH) return -1;
  return 0;  // single pass: the carried state lives in registers
}

extern "C" int32_t catopt_hip_retention_fwd(int32_t dtype, int64_t B, int64_t H, int64_t T,
                                            int64_t d, int64_t chunk, const void* q, const void* k,
                                            const void* v, const float* gamma, float scale, void* o,
                                            void* workspace, int64_t workspace_bytes,
                                            void* stream) {
  (void)workspace;
  if (B < 0 || H < 0 || T < 0 || workspace_bytes < 0) return CATOPT_E_INVAL;
  if (dtype != CATOPT_BF16 || d != HD || chunk != CH) return CATOPT_E_UNSUPPORTED;
  if (T % CH != 0) return CATOPT_E_UNSUPPORTED;
  if (B == 0 || H == 0 || T == 0) return CATOPT_OK;
  if (!q || !k || !v || !gamma || !o) return CATOPT_E_INVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return CATOPT_E_INVAL;
  if (B * H > 0x7fffffffLL / NSL || T / CH > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;
  static bool attr_done = false;
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&retention_scan),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (e != hipSuccess) return set_hip_error(e);
    attr_done = true;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  retention_scan<<<dim3((uint32_t)(B * H * NSL)), dim3(NT), LDS_BYTES, s>>>(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
      static_cast<const uint16_t*>(v), gamma, (int)H, T, scale, static_cast<uint16_t*>(o));
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}
