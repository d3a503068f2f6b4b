// Chunked decayed retention (RetNet) for gfx950, bf16 in / fp32 state.
//
//   o[t] = scale * sum_{s <= t} γ^(t-s) (q[t]·k[s]) v[s]
//
// evaluated chunk-wise with chunk length C = 64 and head dims up to 128.
// Chunk i (rows t = iC + a) takes its diagonal block with decay(γ, C) and
// every strict-lower block through the carried state
//   S_i = sum_{s < iC} γ^(iC - s) k_s ⊗ v_s,   S_{i+1} = γ^C S_i + sum_c γ^(C-c) k_ic ⊗ v_ic,
// so that  o_i = scale * ( (q_i k_iᵀ ⊙ D) v_i + diag(γ^a) q_i S_i ),  D[a][c] = γ^(a-c) (c <= a):
// the K-way block decomposition's algebra, with its rank-1 decay_vec factors
// γ^(a + (i-j)C) · γ^(-c) folded into the state.
//
// Work split.  A head's state is 128 x 128 fp32, and its chunks are a chain,
// so a head runs on one workgroup per T-segment: the chunks split into P
// equal segments (P * B * H about the CU count), and segment s starts from
//   S_start(s) = sum over chunk ranges R before segment s of γ^((c_s - r1(R)) C) W_R,
//   W_R = sum_{i in R} γ^((r1 - 1 - i) C) D_i,   D_i = sum_c γ^(C-c) k_ic ⊗ v_ic.
// Two kernels:
//   retention_state  the W_R of the chunks before the last segment, that
//                    prefix cut into P equal ranges (one workgroup each,
//                    every range split where it crosses a segment start);
//                    reads k and v once more, writes one 64 KB fp32 state
//                    per piece;
//   retention_out    one workgroup per (b, h, segment): sums its start state
//                    from the pieces, then walks the segment's chunks, so q,
//                    k, v and o cross HBM once there and each chunk's q, k, v
//                    tiles cross global->LDS once per head.
// With P = 1 (enough heads to fill the chip) retention_out alone runs, from
// a zero state.
//
// Inside a workgroup (4 waves, 32x32x16 bf16 MFMA, fp32 accumulation) wave w
// owns the v columns dv = 32w .. 32w+31: its state columns S[:, dv] (four
// 32 x 32 tiles over dk) and its output columns.  Products are computed
// transposed (output column = query):
//   X  = S_wᵀ Qᵀ               A = the wave's own S accumulators (bf16),
//                              B = q rows
//   X *= scale γ^a             (per lane: the lane's column is the query a)
//   sᵀ = K Qᵀ  (waves 0-2,     A = k rows, B = q rows; one 32 x 32 tile of
//       one tile each)         the causal 64 x 64 block per wave, decayed
//                              and published as bf16 P through LDS
//   X += Vᵀ (P)                A = v via the transposing LDS read, B = P
//   S  = γ^C S + Kᵀ (γ^(C-c) V)   A = k via the transposing LDS read,
//                              B = v likewise, each lane decaying its own
//                              elements in registers
// The state tile's row order is chosen by the addresses of the transposing k
// read: accumulator register group 8h .. 8h+7 of half g then holds dk
// 16h + 8g .. +7 of the tile, in order, so those registers are exactly the
// A operand of the X product for that dk step (no trip through LDS).  Every
// product over keys takes its keys in the score accumulator's row order
// 8(r/4) + 4g + r%4, so P feeds an MFMA from the accumulator layout.
//
// Two barriers per chunk: one publishes P, the other the chunk's output
// rows, which the waves stage as bf16 in the chunk's own q tile (each wave
// holds 32 of a row's 128 columns) so that they leave as whole 256-byte
// rows at the start of the next chunk.  Tiles reach LDS by direct
// global->LDS loads through buffer resources over the chunk's rows (a ring
// of three stages: chunk i + 2 is loaded into chunk i - 1's stage once its
// rows are out), so rows past T and columns past the head dims read as
// zeros and need no padded copy; output stores go through a buffer resource
// too, and those past T or the head dim are dropped.
#include <type_traits>

#include "common.hpp"

namespace catopt {
namespace {

constexpr int NT = 256;
constexpr int CH = 64;                 // chunk length
constexpr int HD = 128;                // largest head dim (dk, dv); tiles are laid out at 128
constexpr int TILE = CH * HD * 2;      // one [64][128] bf16 tile, 16 KB
constexpr int NSTAGE_C = 3;            // retention_out: stages of (k, q, v)
constexpr int STAGE_C = 3 * TILE;
constexpr int PB_BYTES = 3 * 2 * 64 * 16;   // P: 3 score tiles x 2 key steps x 64 lanes x 16 B
constexpr int OFF_P = NSTAGE_C * STAGE_C;
constexpr int LDS_C = OFF_P + PB_BYTES;
static_assert(LDS_C <= 160 * 1024, "retention_out LDS");
constexpr int NSTAGE_A = 4;            // retention_state: stages of (k, v)
constexpr int STAGE_A = 2 * TILE;
constexpr int LDS_A = NSTAGE_A * STAGE_A;
static_assert(LDS_A <= 160 * 1024, "retention_state LDS");
constexpr int WFLOATS = HD * HD;       // one state piece: 128 x 128 fp32
constexpr int MAXSEG = 8;
constexpr int MAXPIECE = 2 * MAXSEG;
constexpr uint32_t kOOB = 0x80000000u;  // a buffer offset past every range: loads 0, stores dropped

// Segments of a head's chunks and the state pieces before them (the same for
// every head).  Workgroup j of retention_state writes pieces 2j and 2j + 1
// (empty when r0 == r1).
struct SegPlan {
  int nseg;
  int seg[MAXSEG + 1];
  int r0[MAXPIECE];
  int r1[MAXPIECE];
};

typedef __attribute__((ext_vector_type(4))) short s16x4;

// s_waitcnt: vmcnt <= n, lgkmcnt = 0, expcnt not waited on (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(n >= 0 && n < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | ((n >> 4) << 14));
}

// The 16-byte chunk index of a tile row is XOR-ed with a bijection of the
// row's position among 16 consecutive rows (low two bits to bits 2-3, bits
// 2-3 to bits 0-1).  A plain row read (16 consecutive rows, one chunk) hits
// 16 distinct chunk slots, and so does a transposing read (4 consecutive
// rows x 4 adjacent 8-byte pieces per 16 lanes, rows a bank window apart).
__device__ __forceinline__ int kq_swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }
__device__ __forceinline__ int kq_off(int row, int chunk) {  // byte offset in a tile
  return row * (HD * 2) + ((chunk ^ kq_swz(row)) << 4);
}

// Transposing LDS read (ds_read_b64_tr_b16).  Within each 16-lane group, lane
// j (= 4r + a) reads 4 consecutive bf16 at its address; lane i receives, for
// r = 0..3, element i % 4 of lane 4r + i / 4.  With lane 4r + a pointing at
// row base + r, columns c0 + 4 σ(a) .. +3, lane i gets column
// c0 + 4 σ(i / 4) + i % 4 of rows base .. base + 3.
__device__ __forceinline__ s16x4 ds_read_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
}

__device__ __forceinline__ bf16x8 cat8(s16x4 lo, s16x4 hi) {
  const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
  return __builtin_bit_cast(bf16x8, u32x4{a[0], a[1], b[0], b[1]});
}

__device__ __forceinline__ bf16x8 pack8(const f32x16& x, int h) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(x[8 * h + 2 * i], x[8 * h + 2 * i + 1]);
  return __builtin_bit_cast(bf16x8, w);
}

// Per-lane fragment addressing shared by both kernels.
struct Lanes {
  int lane, l32, g, G, jj;
  __device__ Lanes(int tid) {
    lane = tid & 63;
    l32 = lane & 31;
    g = lane >> 5;
    G = lane >> 4;
    jj = lane & 15;
  }
  // key row of the transposing reads for key step u: the lower 4 keys (the
  // upper 4 are 8 rows further)
  __device__ int tr_key(int u) const { return 16 * u + 4 * (G >> 1) + (jj >> 2); }
  // v column of the transposing v read (natural order within the wave's slice)
  __device__ int tr_vcol(int w) const { return 32 * w + 16 * (G & 1) + 4 * (jj & 3); }
  // dk column of the transposing k read for state tile t: the middle two
  // groups of four of every 16 swapped (σ = 0, 2, 1, 3), so that the state
  // accumulator of half g holds dk 16h + 8g .. +7 in registers 8h .. 8h+7
  __device__ int tr_kcol(int t) const {
    const int a = jj & 3;
    const int sa = ((a & 1) << 1) | (a >> 1);
    return 32 * t + 16 * (G & 1) + 4 * sa;
  }
};

// the lower four keys at `row`, the upper four at row + 8 (each row has its
// own swizzle)
__device__ __forceinline__ bf16x8 read_tr_pair(const char* tile, int row, int col) {
  const int c = col >> 3, b = (col & 7) * 2;
  return cat8(ds_read_tr(tile + kq_off(row, c) + b), ds_read_tr(tile + kq_off(row + 8, c) + b));
}

// Global->LDS loads of one [64][128] tile: thread slot i (0..3) covers the
// 16-byte piece s = 256 i + tid, LDS byte 16 s, row s / 16, LDS chunk s % 16,
// which holds global chunk (s % 16) ^ kq_swz(row).  Offsets are bytes from
// the chunk's first row; chunks past the row's width load zeros (kOOB).
__device__ __forceinline__ void tile_offsets(int tid, int width, uint32_t off[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = i * NT + tid;
    const int row = s >> 4, c = (s & 15) ^ kq_swz(row);
    off[i] = 8 * c < width ? (uint32_t)(row * width + 8 * c) * 2u : kOOB;
  }
}

__device__ __forceinline__ void dma_tile(const uint16_t* base, int64_t rows, int width,
                                         const uint32_t off[4], uint32_t lds_wave) {
  const u32x4 r = make_rsrc(base, (uint32_t)(rows * width * 2));
#pragma unroll
  for (int i = 0; i < 4; ++i) dma_buf(r, off[i], lds_wave + i * NT * 16);
}

// Decay factors of a lane's transposed-v elements: element e of the key-step
// u fragment is key 16u + 4g + (e < 4 ? e : e + 4); vf3[e] = γ^(C - key) at
// u = 3, and step u - 1's factors are step u's times γ^16.
__device__ __forceinline__ void v_decay3(const Lanes& L, float lg, bool neg, float vf3[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = 48 + 4 * (L.G >> 1) + (e < 4 ? e : e + 4);
    vf3[e] = pow_k(lg, neg, CH - key);
  }
}

// D update of the four state tiles: S[t] += Kᵀ_t · (f γ^(C-c) V), the chunk's
// k and v tiles in LDS.  The caller scales S beforehand.
__device__ __forceinline__ void state_update(f32x16 S[4], const char* Ks, const char* Vs,
                                             const Lanes& L, int w, const float vf3[8], float g16,
                                             float f, bf16x8 vt[4]) {
  float vf[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) vf[e] = vf3[e] * f;
#pragma unroll
  for (int u = 0; u < 4; ++u) vt[u] = read_tr_pair(Vs, L.tr_key(u), L.tr_vcol(w));
  bf16x8 vd[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int u = 3 - t;  // factors run from step 3 down
    const u32x4 x = __builtin_bit_cast(u32x4, vt[u]);
    u32x4 y;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2)
      y[e2] = pack_bf16x2(__uint_as_float(x[e2] << 16) * vf[2 * e2],
                          __uint_as_float(x[e2] & 0xffff0000u) * vf[2 * e2 + 1]);
    vd[u] = __builtin_bit_cast(bf16x8, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) vf[e] *= g16;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    bf16x8 kt[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) kt[u] = read_tr_pair(Ks, L.tr_key(u), L.tr_kcol(t));
#pragma unroll
    for (int u = 0; u < 4; ++u) S[t] = mfma32x32x16(kt[u], vd[u], S[t]);
  }
}

// One state piece in its register-native layout: float4 index
// ((w * 4 + t) * 4 + r4) * 64 + lane.
__device__ __forceinline__ int64_t piece_f4(int w, int t, int r4, int lane) {
  return ((int64_t)((w * 4 + t) * 4 + r4)) * 64 + lane;
}

// ---------------------------------------------------------------- state pass
__global__ __launch_bounds__(NT, 1) void retention_state(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, const float* __restrict__ gamma,
    int H, int64_t T, int dk, int dv, int BH, SegPlan plan, float* __restrict__ pieces) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int j = blockIdx.x / BH, bh = blockIdx.x % BH;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Lanes L(tid);
  const float gam = gamma[bh % H];
  const float lg = __log2f(fabsf(gam));
  const bool neg = gam < 0.f;
  const float gC = pow_k(lg, neg, CH);
  const float g16 = pow_k(lg, neg, 16);
  float vf3[8];
  v_decay3(L, lg, neg, vf3);
  uint32_t koff[4], voff[4];
  tile_offsets(tid, dk, koff);
  tile_offsets(tid, dv, voff);
  const uint16_t* kh = k + (int64_t)bh * T * dk;
  const uint16_t* vh = v + (int64_t)bh * T * dv;
  const uint32_t lds0 = lds_u32(lds) + w * 1024;

  // the workgroup's pieces, walked backwards (last chunk first) as one list
  const int pa0 = plan.r0[2 * j], pa1 = plan.r1[2 * j];
  const int pb0 = plan.r0[2 * j + 1], pb1 = plan.r1[2 * j + 1];
  const int na = pa1 - pa0, nb = pb1 - pb0, n = na + nb;
  if (n <= 0) return;
  auto chunk_of = [&](int step) { return step < nb ? pb1 - 1 - step : pa1 - 1 - (step - nb); };
  auto issue = [&](int step, int stage) {
    const int ci = chunk_of(step < n ? step : n - 1);
    const int64_t t0 = (int64_t)ci * CH;
    const int64_t rows = T - t0 < CH ? T - t0 : CH;
    const uint32_t sb = lds0 + stage * STAGE_A;
    dma_tile(kh + t0 * dk, rows, dk, koff, sb);
    dma_tile(vh + t0 * dv, rows, dv, voff, sb + TILE);
  };
#pragma unroll
  for (int p = 0; p < NSTAGE_A - 1; ++p) issue(p, p);

  f32x16 S[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) S[t][r] = 0.f;
  float f = 1.f;  // γ^((r1 - 1 - i) C) of the current chunk within its piece
  float* out = pieces + (int64_t)bh * 2 * plan.nseg * WFLOATS;
  auto flush = [&](int piece) {
    f32x4* dst = reinterpret_cast<f32x4*>(out + (int64_t)piece * WFLOATS);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        dst[piece_f4(w, t, r4, L.lane)] = f32x4{S[t][4 * r4], S[t][4 * r4 + 1], S[t][4 * r4 + 2], S[t][4 * r4 + 3]};
#pragma unroll
        for (int e = 0; e < 4; ++e) S[t][4 * r4 + e] = 0.f;
      }
  };
  constexpr int LOADS = 8;  // global->LDS instructions per thread per chunk
  wait_vm_lgkm0<LOADS * (NSTAGE_A - 2)>();
  __syncthreads();
  for (int step = 0; step < n; ++step) {
    const int stage = step % NSTAGE_A;
    issue(step + NSTAGE_A - 1, (step + NSTAGE_A - 1) % NSTAGE_A);
    const char* Ks = lds + stage * STAGE_A;
    bf16x8 vt[4];
    state_update(S, Ks, Ks + TILE, L, w, vf3, g16, f, vt);
    f *= gC;
    if (step == nb - 1) {  // piece b (the later one) is complete
      flush(2 * j + 1);
      f = 1.f;
    }
    // the next chunk's tiles have landed once no more than the two younger
    // chunks' loads remain (piece b's stores, younger still, only make the
    // wait stricter)
    wait_vm_lgkm0<LOADS * (NSTAGE_A - 2)>();
    __syncthreads();
  }
  flush(2 * j);
}

// --------------------------------------------------------------- output pass
template <int ROLE>  // 0..2: the score tile (kb, qb) = (0,0), (0,1), (1,1); 3: none
__device__ __forceinline__ void out_segment(
    char* lds, const uint16_t* qh, const uint16_t* kh, const uint16_t* vh, uint16_t* oh, int64_t T,
    int dk, int dv, float scale, float lg, bool neg, int c0, int c1, f32x16 S[4], const Lanes& L, int w, int tid) {
  constexpr bool SCORE = ROLE < 3;
  constexpr int KB = ROLE == 2 ? 1 : 0;
  constexpr int QB = ROLE == 0 ? 0 : 1;
  const float gC = pow_k(lg, neg, CH);
  const float g16 = pow_k(lg, neg, 16);
  float vf3[8];
  v_decay3(L, lg, neg, vf3);
  float gq[2];  // scale γ^a of this lane's query column in each query tile
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) gq[qb] = scale * pow_k(lg, neg, 32 * qb + L.l32);
  float dec[16];  // scale γ^(a - c) of the score tile's entries (0 above the diagonal)
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int c = 32 * KB + acc_row(r, L.g), a = 32 * QB + L.l32;
    dec[r] = (SCORE && c <= a) ? scale * pow_k(lg, neg, a - c) : 0.f;
  }
  uint32_t koff[4], voff[4];
  tile_offsets(tid, dk, koff);
  tile_offsets(tid, dv, voff);
  const uint32_t lds0 = lds_u32(lds) + w * 1024;
  auto issue = [&](int ci, int stage) {
    const int64_t t0 = (int64_t)ci * CH;
    const int64_t rows = T - t0 < CH ? T - t0 : CH;
    const uint32_t sb = lds0 + stage * STAGE_C;
    dma_tile(kh + t0 * dk, rows, dk, koff, sb);
    dma_tile(qh + t0 * dk, rows, dk, koff, sb + TILE);
    dma_tile(vh + t0 * dv, rows, dv, voff, sb + 2 * TILE);
  };
#pragma unroll
  for (int p = 0; p < NSTAGE_C - 1; ++p) issue(min(c0 + p, c1 - 1), p);
  constexpr int LOADS = 12;  // global->LDS instructions per thread per chunk
  constexpr int STORES = 4;  // output row stores per thread per chunk

  // A chunk's output rows are staged as bf16 in the q tile of its own stage
  // (free once every wave has read its q fragments), laid out as the tiles
  // are, then each 16-lane group stores one whole 256-byte row: thread
  // tid covers rows tid / 16 + 16 j, 16-byte column piece tid % 16.  Rows
  // past T and pieces past dv are dropped by the buffer range.
  uint32_t soff[4];
  {
    const int pc = tid & 15;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = (tid >> 4) + 16 * j;
      soff[j] = 8 * pc < dv ? (uint32_t)(row * dv + 8 * pc) * 2u : kOOB;
    }
  }
  auto store_rows = [&](int ci, const char* Os) {
    const int64_t t0 = (int64_t)ci * CH;
    const int64_t rows = T - t0 < CH ? T - t0 : CH;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(oh + t0 * dv, (short)0, (int)(rows * dv * 2), 0x00020000);
    u32x4 val[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      val[j] = *reinterpret_cast<const u32x4*>(Os + kq_off((tid >> 4) + 16 * j, tid & 15));
#pragma unroll
    for (int j = 0; j < 4; ++j) __builtin_amdgcn_raw_buffer_store_b128(val[j], r, (int)soff[j], 0, 0);
  };
  // this wave's 32 output columns of the chunk into the staging rows: lane
  // (query 32 qb + l32, half g) holds dv = 32 w + 8 p + 4 g .. +3 in
  // registers 4p .. 4p+3
  auto stage_out = [&](char* Os, const f32x16 X[2]) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int p = 0; p < 4; ++p)
        *reinterpret_cast<u32x2*>(Os + kq_off(32 * qb + L.l32, 4 * w + p) + 8 * L.g) =
            u32x2{pack_bf16x2(X[qb][4 * p], X[qb][4 * p + 1]), pack_bf16x2(X[qb][4 * p + 2], X[qb][4 * p + 3])};
  };

  bf16x8 sbf[4][2];  // the state as the X product's A operand (bf16)
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    sbf[t][0] = pack8(S[t], 0);
    sbf[t][1] = pack8(S[t], 1);
  }
  wait_vm_lgkm0<LOADS * (NSTAGE_C - 2)>();
  __syncthreads();

  // One chunk, two barriers.  Before barrier A: the previous chunk's staged
  // rows go out, then this chunk's fragments, scores, X = Sᵀ Q and the state
  // update; P is published.  After it: the next-but-one chunk's loads go to
  // the previous chunk's stage (its rows have been read), then P·V finishes
  // X and the rows are staged.  Barrier B: staged rows and the next chunk's
  // tiles in place.
  auto chunk = [&](int ci, auto stage_tag) {
    constexpr int cur = decltype(stage_tag)::value;
    constexpr int prev = (cur + NSTAGE_C - 1) % NSTAGE_C;
    char* Ks = lds + cur * STAGE_C;
    char* Qs = Ks + TILE;
    const char* Vs = Qs + TILE;
    const bool first = ci == c0;
    if (!first) store_rows(ci - 1, lds + prev * STAGE_C + TILE);

    // ---- q rows (B operand of X and of the scores)
    bf16x8 qf[2][8];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int jq = 0; jq < 8; ++jq)
        qf[qb][jq] = *reinterpret_cast<const bf16x8*>(Qs + kq_off(32 * qb + L.l32, 2 * jq + L.g));
    f32x16 X[2], sa;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      X[0][r] = 0.f;
      X[1][r] = 0.f;
      sa[r] = 0.f;
    }
    if (SCORE) {
      bf16x8 kf[8];
#pragma unroll
      for (int jq = 0; jq < 8; ++jq)
        kf[jq] = *reinterpret_cast<const bf16x8*>(Ks + kq_off(32 * KB + L.l32, 2 * jq + L.g));
#pragma unroll
      for (int jq = 0; jq < 8; ++jq) sa = mfma32x32x16(kf[jq], qf[QB][jq], sa);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        X[0] = mfma32x32x16(sbf[t][h], qf[0][2 * t + h], X[0]);
        X[1] = mfma32x32x16(sbf[t][h], qf[1][2 * t + h], X[1]);
      }

    // ---- state update (S_{i+1} = γ^C S_i + D_i); vt keeps this chunk's v
    bf16x8 vt[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) S[t][r] *= gC;
    state_update(S, Ks, Vs, L, w, vf3, g16, 1.f, vt);

    // ---- P published (barrier A), then the loads two chunks ahead
    if (SCORE) {
      char* pw = lds + OFF_P + (2 * ROLE) * 1024 + L.lane * 16;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4 pk;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          pk[i] = pack_bf16x2(sa[8 * h + 2 * i] * dec[8 * h + 2 * i], sa[8 * h + 2 * i + 1] * dec[8 * h + 2 * i + 1]);
        *reinterpret_cast<u32x4*>(pw + h * 1024) = pk;
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      sbf[t][0] = pack8(S[t], 0);
      sbf[t][1] = pack8(S[t], 1);
    }
    wait_vm_lgkm0<63>();  // this wave's P written and its LDS reads returned
    __syncthreads();
    issue(min(ci + NSTAGE_C - 1, c1 - 1), prev);

    // ---- X = scale γ^a X + P·V, staged as rows in this chunk's q tile
    {
      const char* pb = lds + OFF_P + L.lane * 16;
      bf16x8 pf[6];
#pragma unroll
      for (int i = 0; i < 6; ++i) pf[i] = *reinterpret_cast<const bf16x8*>(pb + i * 1024);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int r = 0; r < 16; ++r) X[qb][r] *= gq[qb];
      // P fragment (tile tt, key step h) sits at index 2 tt + h
      X[0] = mfma32x32x16(vt[0], pf[0], X[0]);
      X[0] = mfma32x32x16(vt[1], pf[1], X[0]);
      X[1] = mfma32x32x16(vt[0], pf[2], X[1]);
      X[1] = mfma32x32x16(vt[1], pf[3], X[1]);
      X[1] = mfma32x32x16(vt[2], pf[4], X[1]);
      X[1] = mfma32x32x16(vt[3], pf[5], X[1]);
      stage_out(Qs, X);
    }
    // chunk ci+1's tiles have landed once no more than this chunk's loads
    // (issued above) and the row stores issued before them remain
    if (first)
      wait_vm_lgkm0<LOADS>();
    else
      wait_vm_lgkm0<LOADS + STORES>();
    __syncthreads();
  };
  static_assert(NSTAGE_C == 3, "the chunk loop below runs three stages");
  for (int ci = c0; ci < c1; ci += 3) {
    chunk(ci, std::integral_constant<int, 0>{});
    if (ci + 1 < c1) chunk(ci + 1, std::integral_constant<int, 1>{});
    if (ci + 2 < c1) chunk(ci + 2, std::integral_constant<int, 2>{});
  }
  store_rows(c1 - 1, lds + ((c1 - 1 - c0) % NSTAGE_C) * STAGE_C + TILE);
  __builtin_amdgcn_s_waitcnt(0);  // the repeat loads past the segment's last chunk have landed
}

__global__ __launch_bounds__(NT, 1) void retention_out(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ gamma, int H, int64_t T, int dk, int dv, float scale, int BH,
    SegPlan plan, const float* __restrict__ pieces, uint16_t* __restrict__ o) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int s = blockIdx.x / BH, bh = blockIdx.x % BH;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Lanes L(tid);
  const float gam = gamma[bh % H];
  const float lg = __log2f(fabsf(gam));
  const bool neg = gam < 0.f;
  const int c0 = plan.seg[s], c1 = plan.seg[s + 1];
  if (c0 >= c1) return;

  // the segment's start state: the pieces that end at or before its start,
  // each decayed to it
  f32x16 S[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) S[t][r] = 0.f;
  if (s > 0) {
    const float* ph = pieces + (int64_t)bh * 2 * plan.nseg * WFLOATS;
    for (int p = 0; p < 2 * plan.nseg; ++p) {
      if (plan.r0[p] >= plan.r1[p] || plan.r1[p] > c0) continue;
      const float fct = pow_k(lg, neg, (c0 - plan.r1[p]) * CH);
      const f32x4* src = reinterpret_cast<const f32x4*>(ph + (int64_t)p * WFLOATS);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 x = src[piece_f4(w, t, r4, L.lane)];
#pragma unroll
          for (int e = 0; e < 4; ++e) S[t][4 * r4 + e] += fct * x[e];
        }
    }
  }
  const int64_t hb = (int64_t)bh * T;
  const uint16_t* qh = q + hb * dk;
  const uint16_t* kh = k + hb * dk;
  const uint16_t* vh = v + hb * dv;
  uint16_t* oh = o + hb * dv;
  // wave roles: waves 0-2 each take one score tile of the causal block
  if (w == 0)
    out_segment<0>(lds, qh, kh, vh, oh, T, dk, dv, scale, lg, neg, c0, c1, S, L, w, tid);
  else if (w == 1)
    out_segment<1>(lds, qh, kh, vh, oh, T, dk, dv, scale, lg, neg, c0, c1, S, L, w, tid);
  else if (w == 2)
    out_segment<2>(lds, qh, kh, vh, oh, T, dk, dv, scale, lg, neg, c0, c1, S, L, w, tid);
  else
    out_segment<3>(lds, qh, kh, vh, oh, T, dk, dv, scale, lg, neg, c0, c1, S, L, w, tid);
}

// Segments per head: about one workgroup per CU in all, at least two chunks
// per segment, at most MAXSEG.
int n_segments(int64_t BH, int64_t nch, int n_cu) {
  int64_t p = (n_cu + BH - 1) / BH;
  if (p > MAXSEG) p = MAXSEG;
  if (p > nch / 2) p = nch / 2;
  return p < 1 ? 1 : (int)p;
}

SegPlan make_plan(int P, int64_t nch) {
  SegPlan pl{};
  pl.nseg = P;
  for (int s = 0; s <= P; ++s) pl.seg[s] = (int)((s * nch) / P);
  // the state prefix (every chunk before the last segment) in P equal
  // ranges, each split where it crosses a segment start
  const int na = pl.seg[P - 1];
  for (int j = 0; j < P; ++j) {
    const int a0 = (int)(((int64_t)j * na) / P), a1 = (int)(((int64_t)(j + 1) * na) / P);
    int cut = a1;
    for (int s = 1; s < P; ++s)
      if (pl.seg[s] > a0 && pl.seg[s] < a1) {
        cut = pl.seg[s];
        break;
      }
    pl.r0[2 * j] = a0;
    pl.r1[2 * j] = cut;
    pl.r0[2 * j + 1] = cut;
    pl.r1[2 * j + 1] = a1;
  }
  for (int p = 2 * P; p < MAXPIECE; ++p) pl.r0[p] = pl.r1[p] = 0;
  return pl;
}

// A range crosses at most one segment start (ranges are shorter than
// segments); the plan is rejected otherwise.
bool plan_ok(const SegPlan& pl) {
  for (int j = 0; j < pl.nseg; ++j)
    for (int s = 1; s < pl.nseg; ++s)
      if (pl.seg[s] > pl.r0[2 * j + 1] && pl.seg[s] < pl.r1[2 * j + 1]) return false;
  return true;
}

int cu_count_of_current_device(int* out) {
  static int cache[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_hip_error(e);
  int n = dev >= 0 && dev < 64 ? cache[dev] : 0;
  if (n == 0) {
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return set_hip_error(e);
    if (n < 1) n = 1;
    if (dev >= 0 && dev < 64) cache[dev] = n;
  }
  *out = n;
  return CATOPT_OK;
}

bool dims_ok(int64_t dk, int64_t dv) {
  return dk >= 8 && dv >= 8 && dk <= HD && dv <= HD && dk % 8 == 0 && dv % 8 == 0;
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int64_t catopt_hip_retention_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t d,
                                                        int64_t chunk) {
  if (B < 0 || H < 0 || T < 0 || !dims_ok(d, d) || chunk != CH) return -1;
  const int64_t BH = B * H, nch = (T + CH - 1) / CH;
  if (BH == 0 || nch == 0) return 0;
  // the current device's segment count; without a device, the most any
  // device can take (the bound on segments alone)
  int n_cu = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    n_cu = 0x3fffffff;
  const int P = n_segments(BH, nch, n_cu);
  if (P == 1) return 0;
  return BH * 2 * P * WFLOATS * (int64_t)sizeof(float);  // two state pieces per range
}

namespace catopt {
// fp32 operands (retention_f32.hip): d a multiple of 4 up to 128, any T.
int32_t retention_f32_launch(int64_t B, int64_t H, int64_t T, int64_t d, const float* q, const float* k,
                             const float* v, const float* gamma, float scale, float* o, hipStream_t s);
}  // namespace catopt

extern "C" int32_t catopt_hip_retention_fwd(int32_t dtype, int64_t B, int64_t H, int64_t T,
                                            int64_t d, int64_t chunk, const void* q, const void* k,
                                            const void* v, const float* gamma, float scale, void* o,
                                            void* workspace, int64_t workspace_bytes,
                                            void* stream) {
  if (B < 0 || H < 0 || T < 0 || workspace_bytes < 0) return CATOPT_E_INVAL;
  if (dtype == CATOPT_F32) {  // no workspace: the state stays in registers
    if (d < 1 || d > 128 || d % 4 || chunk != CH) return CATOPT_E_UNSUPPORTED;
    if (B == 0 || H == 0 || T == 0) return CATOPT_OK;
    if (!q || !k || !v || !gamma || !o) return CATOPT_E_INVAL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return CATOPT_E_INVAL;
    return retention_f32_launch(B, H, T, d, static_cast<const float*>(q), static_cast<const float*>(k),
                                static_cast<const float*>(v), gamma, scale, static_cast<float*>(o),
                                static_cast<hipStream_t>(stream));
  }
  if (dtype != CATOPT_BF16 || !dims_ok(d, d) || chunk != CH) return CATOPT_E_UNSUPPORTED;
  if (B == 0 || H == 0 || T == 0) return CATOPT_OK;
  if (!q || !k || !v || !gamma || !o) return CATOPT_E_INVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return CATOPT_E_INVAL;
  const int64_t BH = B * H, nch = (T + CH - 1) / CH;
  // 32-bit buffer ranges per chunk, int chunk indices, grid within 2^31
  if (BH * MAXSEG > 0x7fffffffLL || nch > 0x3fffffffLL) return CATOPT_E_UNSUPPORTED;
  int n_cu = 0;
  int32_t st = cu_count_of_current_device(&n_cu);
  if (st != CATOPT_OK) return st;
  const int P = n_segments(BH, nch, n_cu);
  const SegPlan plan = make_plan(P, nch);
  if (!plan_ok(plan)) return CATOPT_E_UNSUPPORTED;
  if (P > 1) {
    if (!workspace || !aligned16(workspace)) return CATOPT_E_INVAL;
    if (workspace_bytes < BH * 2 * P * WFLOATS * (int64_t)sizeof(float)) return CATOPT_E_WORKSPACE;
  }
  static bool attr_done = false;
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&retention_out),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS_C);
    if (e != hipSuccess) return set_hip_error(e);
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&retention_state),
                            hipFuncAttributeMaxDynamicSharedMemorySize, LDS_A);
    if (e != hipSuccess) return set_hip_error(e);
    attr_done = true;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto qp = static_cast<const uint16_t*>(q);
  auto kp = static_cast<const uint16_t*>(k);
  auto vp = static_cast<const uint16_t*>(v);
  float* pieces = static_cast<float*>(workspace);
  if (P > 1) {
    retention_state<<<dim3((uint32_t)(P * BH)), dim3(NT), LDS_A, s>>>(kp, vp, gamma, (int)H, T, (int)d,
                                                                      (int)d, (int)BH, plan, pieces);
    CATOPT_LAUNCH_CHECK();
  }
  retention_out<<<dim3((uint32_t)(P * BH)), dim3(NT), LDS_C, s>>>(qp, kp, vp, gamma, (int)H, T, (int)d,
                                                                  (int)d, scale, (int)BH, plan, pieces,
                                                                  static_cast<uint16_t*>(o));
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}
