// bf16 "NT" GEMM on gfx950 MFMA with fused epilogues.
//
//   C[m, n] = epi( sum_k A[m, k] * B[n, k] )
//
// A is the activation (rows of length K, K contiguous), B the weight in
// nn.Linear layout (out_features x in_features, K contiguous): both operands
// are K-contiguous, which is the layout the 32x32x16 MFMA consumes directly
// (each lane supplies 8 consecutive k of one row/column).
//
// Tiling: 256x256 block tile, BK = 64, 8 waves in a 2x4 grid (two per
// SIMD), each wave a 128x64 sub-tile = 4x2 MFMA blocks.  Tiles reach LDS by
// direct buffer->LDS loads (buffer_load_dwordx4 ... lds) through buffer
// resources over the tile's rows: one precomputed 32-bit offset per load slot
// plus the K offset, so a tile's loads cost no 64-bit address arithmetic; no
// register staging, no LDS store instructions.  A ring of LDS stages (two of 64 KB): the loads
// of K tile t+1 are issued before the MFMAs of tile t, one barrier per K
// tile.  Within a tile the fragments of k-step s+1 are read before the MFMAs
// of k-step s, and the last k-step's MFMAs are issued after the barrier,
// behind the next tile's first reads.  (Measured on MI355X: shallower K
// tiles with a deeper ring lose more to the extra barriers than they gain
// in loads in flight; 128x128 wave tiles at one wave per SIMD lose to the
// two-waves-per-SIMD layout.)  The 16-byte chunk index of each LDS row is
// XOR-swizzled so a fragment read's 16 rows per pass hit 16 bank groups.
//
// Edges: rows past M (A) or N (B) load a clamped, valid row and are never
// stored; in a K tail (K % 64 != 0, K % 8 == 0) the chunks past K read the
// next row's head or, past the operand's end, the buffer range check's zero,
// and are zeroed in LDS before they are read.  Every offset within a tile's
// rows must fit in 31 bits (checked on the host).
//
// Paired epilogues (SILU_MUL / GLU): the B tile holds 128 rows of the first
// projection and the 128 matching rows of the second (row n and row n + N of
// the concatenated weight), so every wave owns both halves of its output
// columns and the gate is applied in registers — the chunk/silu/mul of the
// SWIGLU_FUSE form never touch HBM.
//
// Block-to-tile mapping is XCD-aware: the hardware deals workgroups round
// robin over 8 XCDs, so each XCD is given a contiguous range of logical tiles
// (grouped 8 M-tiles at a time), which march through K together and share
// that XCD's L2.
#include "common.hpp"

namespace catopt {
namespace {

#ifndef CATOPT_GEMM_BK
#define CATOPT_GEMM_BK 64
#endif
#ifndef CATOPT_GEMM_STAGES
#define CATOPT_GEMM_STAGES 2
#endif
constexpr int BM = 256, BN = 256, BK = CATOPT_GEMM_BK;
constexpr int NSTAGE = CATOPT_GEMM_STAGES;
#ifndef CATOPT_GEMM_NWN
#define CATOPT_GEMM_NWN 4
#endif
constexpr int NWN = CATOPT_GEMM_NWN;    // waves along N (2 along M)
constexpr int NT = 128 * NWN;           // threads per block
constexpr int WCOLS = BN / NWN;         // output columns per wave (B rows)
constexpr int TJ = WCOLS / 32;          // 32-wide MFMA blocks per wave along N
constexpr int CPR = BK / 8;             // 16-byte chunks per tile row
constexpr int RPB = 256 / (BK * 2);     // tile rows per 256 bytes (one pass of the LDS banks)
constexpr int TILE_BYTES = BM * BK * 2;                 // one operand tile (A or B)
constexpr int STAGE_BYTES = 2 * TILE_BYTES;             // A then B
constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES;
constexpr int SLOTS_PER_THREAD = (BM * BK / 8) / NT;    // 16-byte slots per thread per operand
static_assert(SLOTS_PER_THREAD >= 1 && (BM * BK / 8) % NT == 0, "tile / thread mismatch");
static_assert(NSTAGE >= 2 && LDS_BYTES <= 160 * 1024, "LDS ring does not fit");
static_assert(BK % 16 == 0 && RPB >= 1 && CPR * RPB == 16, "row geometry");

typedef __attribute__((address_space(3))) void* lds_ptr;

// The 16-byte chunk index is XOR-swizzled by the row's position among the 16
// consecutive rows that one 16-lane pass of a fragment read touches, so those
// 16 rows land on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int chunk_swizzle(int row) { return (row / RPB) % CPR; }
__device__ __forceinline__ int swz(int row, int chunk) {  // byte offset of (row, chunk) in a tile
  return row * (BK * 2) + ((chunk ^ chunk_swizzle(row)) << 4);
}

// s_waitcnt: vmcnt <= n, lgkmcnt = 0, expcnt not waited on (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(n >= 0 && n < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | ((n >> 4) << 14));
}

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt not waited on).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14)); }

struct TileMap {
  int tm, tn;
};

__device__ __forceinline__ TileMap map_tile(int tiles_m, int tiles_n) {
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) {
    const int xcd = bid & 7, loc = bid >> 3;
    bid = xcd * (nb >> 3) + loc;
  }
  constexpr int GM = 8;
  const int per_group = GM * tiles_n;
  const int group = bid / per_group;
  const int first_m = group * GM;
  const int gsize = min(tiles_m - first_m, GM);
  const int in_group = bid - group * per_group;
  TileMap t;
  t.tm = first_m + in_group % gsize;
  t.tn = in_group / gsize;
  return t;
}

template <int EPI>
__global__ __launch_bounds__(NT, 1) void gemm_bf16_nt(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B, int64_t ldb,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ bias2,
    uint16_t* __restrict__ C, int64_t ldc, int M, int N, int K, int tiles_m, int tiles_n,
    int64_t sA, int64_t sB, int64_t sC) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  A += (int64_t)blockIdx.y * sA;
  B += (int64_t)blockIdx.y * sB;
  C += (int64_t)blockIdx.y * sC;
  constexpr bool PAIRED = (EPI == CATOPT_EPI_SILU_MUL || EPI == CATOPT_EPI_GLU);
  const TileMap tile = map_tile(tiles_m, tiles_n);
  const int m0 = tile.tm * BM;
  // n0: first output column of this tile; B rows for the tile start at n0
  // (and at N + n0 for the second projection of a paired epilogue).
  const int n0 = tile.tn * (PAIRED ? BN / 2 : BN);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / NWN, wn = wave % NWN;
  const int l32 = lane & 31, g = lane >> 5;

  // This thread's load slots: slot s = i*NT + wave*64 + lane of a tile is
  // (row s/8, swizzled chunk s%8); the global row is clamped to a valid one.
  // Buffer resources over this tile's rows: 32-bit offsets from the tile's
  // first row (rows past M / N clamp to the last valid one); a paired tile
  // reads its up rows through a second resource N rows further on.  The K
  // offset rides in the per-lane offset, which the range check covers: a
  // chunk past K of the tail tile reads the next row's head (in bounds) or,
  // past the operand's last element, zero; zero_k_tail clears those chunks.
  const uint16_t* Ab = A + (int64_t)m0 * lda;
  // num_records covers this tile's rows only (at most BM rows from the
  // first): the host check that every in-tile offset fits 31 bits then
  // bounds it too, however large the rest of the operand is
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)Ab, (short)0, (int)(((int64_t)min(M - 1 - m0, BM - 1) * lda + K) * 2), 0x00020000);
  const uint16_t* Bb0 = B + (int64_t)n0 * ldb;
  const int b_rec = (int)(((int64_t)min(N - 1 - n0, (PAIRED ? BN / 2 : BN) - 1) * ldb + K) * 2);
  const __amdgpu_buffer_rsrc_t rb0 = __builtin_amdgcn_make_buffer_rsrc((void*)Bb0, (short)0, b_rec, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb1 = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(Bb0 + (PAIRED ? (int64_t)N * ldb : 0)), (short)0, b_rec, 0x00020000);
  uint32_t a_vo[SLOTS_PER_THREAD], b_vo[SLOTS_PER_THREAD];
  // slot i covers tile rows [i * NT / CPR, (i + 1) * NT / CPR): whether it
  // reads up rows is known at compile time, so the resource stays uniform
  static_assert(128 % (NT / CPR) == 0, "a load slot straddles the gate / up halves");
#pragma unroll
  for (int i = 0; i < SLOTS_PER_THREAD; ++i) {
    const int s = i * NT + wave * 64 + lane;
    const int r = s / CPR, cp = s % CPR;
    const int chunk = cp ^ chunk_swizzle(r);
    const int am = min(r, M - 1 - m0);
    const int bn = PAIRED ? min(r & 127, N - 1 - n0) : min(r, N - 1 - n0);
    a_vo[i] = (uint32_t)(((int64_t)am * lda + chunk * 8) * 2);
    b_vo[i] = (uint32_t)(((int64_t)bn * ldb + chunk * 8) * 2);
  }

  const int ktiles = (K + BK - 1) / BK;
  const bool k_tail = (K % BK) != 0;

  auto issue = [&](int kt, int stage) {
    const uint32_t koff = (uint32_t)kt * (BK * 2);
    char* sa = lds + stage * STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < SLOTS_PER_THREAD; ++i) {
      char* dst = sa + (i * NT + wave * 64) * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr)dst, 16, a_vo[i] + koff, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds((PAIRED && i * (NT / CPR) >= 128) ? rb1 : rb0,
                                               (lds_ptr)(dst + TILE_BYTES), 16,
                                               b_vo[i] + koff, 0, 0, 0);
    }
  };
  // zero the chunks past K of the tail tile (after its loads landed)
  auto zero_k_tail = [&](int kt, int stage) {
    const int k0 = kt * BK;
    char* sa = lds + stage * STAGE_BYTES;
    for (int s = tid; s < 2 * BM * CPR; s += NT) {
      const int t = s / (BM * CPR), rem = s % (BM * CPR);  // operand, slot
      const int r = rem / CPR, cp = rem % CPR;
      const int chunk = cp ^ chunk_swizzle(r);
      if (k0 + chunk * 8 >= K) *reinterpret_cast<u32x4*>(sa + t * TILE_BYTES + rem * 16) = u32x4{0, 0, 0, 0};
    }
  };

  f32x16 acc[4][TJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // B-tile row of the wave's column block j (paired: the first TJ/2 blocks
  // are gate rows, the rest the matching up rows 128 further down).
  auto brow = [&](int j) {
    return PAIRED ? (j / (TJ / 2)) * 128 + wn * (WCOLS / 2) + (j % (TJ / 2)) * 32 : wn * WCOLS + j * 32;
  };

  // Prologue: tiles 0 .. NSTAGE-2 in flight.  Every thread issues the same
  // number of loads per tile slot (slots past the last tile reload it into a
  // stage nobody reads), so "all but the newest NSTAGE-2 tiles landed" is
  // one fixed vmcnt.
  constexpr int LOADS_PER_TILE = 2 * SLOTS_PER_THREAD;
#pragma unroll
  for (int p = 0; p < NSTAGE - 1; ++p) issue(min(p, ktiles - 1), p);
  wait_vm_lgkm0<LOADS_PER_TILE * (NSTAGE - 2)>();
  __syncthreads();
  if (k_tail && ktiles == 1) {
    zero_k_tail(0, 0);
    __syncthreads();
  }

  // Fragment registers: two sets, k-step ks of a tile uses set ks & 1.  The
  // fragments of k-step ks+1 are read before the MFMAs of k-step ks are
  // issued, and the last k-step's MFMAs are issued after the barrier that
  // publishes the next tile, behind that tile's first fragment reads, so the
  // matrix cores keep working across the barrier.
  constexpr int KS = BK / 16;
  static_assert(KS % 2 == 0, "the k-step register sets alternate within a tile");
  bf16x8 af[2][4], bfr[2][TJ];
  auto read_frags = [&](int stage, int ks, int set) {
    const char* As = lds + stage * STAGE_BYTES;
    const char* Bs = As + TILE_BYTES;
    const int chunk = 2 * ks + g;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[set][i] = *reinterpret_cast<const bf16x8*>(As + swz(wm * 128 + i * 32 + l32, chunk));
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      bfr[set][j] = *reinterpret_cast<const bf16x8*>(Bs + swz(brow(j) + l32, chunk));
  };
  auto mfmas = [&](int set) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j] = mfma32x32x16(af[set][i], bfr[set][j], acc[i][j]);
  };

  read_frags(0, 0, 0);
  int cur = 0;
  for (int kt = 0; kt < ktiles; ++kt) {
    // the stage tile kt-1 used receives tile kt + NSTAGE - 1 (its last reads
    // happened before the barrier that ended iteration kt-1)
    issue(min(kt + NSTAGE - 1, ktiles - 1), cur == 0 ? NSTAGE - 1 : cur - 1);
    const int nxt = cur + 1 == NSTAGE ? 0 : cur + 1;
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      // k-step ks's fragments (read one step earlier) have landed before the
      // next step's reads go out: the MFMAs below then wait on nothing, where
      // the compiler's own wait before them would also cover the new reads.
      wait_lgkm0();
      read_frags(cur, ks + 1, (ks + 1) & 1);
      mfmas(ks & 1);
      // LLVM's single-wave GEMM strategy spreads the reads among the MFMAs
      // (measured +1% over issuing the reads as one batch ahead of them)
      __builtin_amdgcn_iglp_opt(1);
      __builtin_amdgcn_sched_barrier(0);
    }
    // the last k-step's fragments have landed on both paths below, so the
    // MFMAs after the branch do not wait for the next tile's first reads
    wait_lgkm0();
    if (kt + 1 < ktiles) {
      // loads land in issue order: all but the newest NSTAGE-2 tiles means
      // tile kt+1 is in place
      wait_vm_lgkm0<LOADS_PER_TILE * (NSTAGE - 2)>();
      __syncthreads();
      if (k_tail && kt + 2 == ktiles) {
        zero_k_tail(kt + 1, nxt);
        __syncthreads();
      }
      read_frags(nxt, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mfmas((KS - 1) & 1);
    __builtin_amdgcn_sched_barrier(0);
    cur = nxt;
  }
  __builtin_amdgcn_s_waitcnt(0);  // drain the reloads past the last tile

  // Epilogue: lane owns output column (l32) of each 32-wide block and 16 rows.
  if (PAIRED) {
#pragma unroll
    for (int j = 0; j < TJ / 2; ++j) {
      const int n = n0 + wn * (WCOLS / 2) + j * 32 + l32;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * 128 + i * 32 + acc_row(r, g);
          if (m >= M) continue;
          const float a = acc[i][j][r], b = acc[i][j + TJ / 2][r];
          const float o = (EPI == CATOPT_EPI_SILU_MUL) ? silu_f(a) * b : a * sigmoid_f(b);
          C[(int64_t)m * ldc + n] = f32_to_bf16(o);
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int n = n0 + wn * WCOLS + j * 32 + l32;
      if (n >= N) continue;
      float badd = 0.f;
      if (EPI == CATOPT_EPI_BIAS || EPI == CATOPT_EPI_BIAS_ADD2) badd = bf16_to_f32(bias[n]);
      float badd2 = 0.f;
      if (EPI == CATOPT_EPI_BIAS_ADD2) badd2 = bf16_to_f32(bias2[n]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * 128 + i * 32 + acc_row(r, g);
          if (m >= M) continue;
          float o = acc[i][j][r];
          if (EPI == CATOPT_EPI_BIAS || EPI == CATOPT_EPI_BIAS_ADD2) o += badd;
          if (EPI == CATOPT_EPI_BIAS_ADD2) o += badd2;
          C[(int64_t)m * ldc + n] = f32_to_bf16(o);
        }
      }
    }
  }
}

template <int EPI>
int32_t launch(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb,
               const uint16_t* bias, const uint16_t* bias2, uint16_t* C, int64_t ldc, int M,
               int N, int K, int64_t batch, int64_t sA, int64_t sB, int64_t sC, hipStream_t s) {
  constexpr bool PAIRED = (EPI == CATOPT_EPI_SILU_MUL || EPI == CATOPT_EPI_GLU);
  static bool attr_done = false;  // idempotent; benign race (same value written)
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_bf16_nt<EPI>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (e != hipSuccess) return set_hip_error(e);
    attr_done = true;
  }
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + (PAIRED ? BN / 2 : BN) - 1) / (PAIRED ? BN / 2 : BN);
  const int64_t nblocks = (int64_t)tiles_m * tiles_n;
  if (nblocks > 0x7fffffff || batch > 65535) return CATOPT_E_UNSUPPORTED;
  gemm_bf16_nt<EPI><<<dim3((uint32_t)nblocks, (uint32_t)batch), dim3(NT), LDS_BYTES, s>>>(
      A, lda, B, ldb, bias, bias2, C, ldc, M, N, K, tiles_m, tiles_n, sA, sB, sC);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

}  // namespace

// Fast-path predicate shared with the dispatcher in gemm.hip.
bool gemm_bf16_nt_fast_ok(int64_t M, int64_t N, int64_t K, const void* x, int64_t ldx,
                          const void* w, int64_t ldw, const void* y, int64_t ldy) {
  // buffer offsets within one tile's rows: (255 * ld + K) * 2 bytes < 2^31
  const bool offsets_fit = (256 * (ldx > ldw ? ldx : ldw) + K) * 2 < (1LL << 31);
  return M > 0 && N > 0 && K > 0 && M < (1LL << 31) && N < (1LL << 30) && K < (1LL << 31) &&
         K % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldx >= K && ldw >= K && offsets_fit &&
         aligned16(x) && aligned16(w) && ldy >= 1 && y != nullptr;
}

int32_t gemm_bf16_nt_launch(int32_t epi, int64_t M, int64_t N, int64_t K, const void* x,
                            int64_t ldx, const void* w, int64_t ldw, const void* bias,
                            const void* bias2, void* y, int64_t ldy, int64_t batch,
                            int64_t sA, int64_t sB, int64_t sC, hipStream_t s) {
  auto A = static_cast<const uint16_t*>(x);
  auto B = static_cast<const uint16_t*>(w);
  auto b1 = static_cast<const uint16_t*>(bias);
  auto b2 = static_cast<const uint16_t*>(bias2);
  auto C = static_cast<uint16_t*>(y);
  switch (epi) {
    case CATOPT_EPI_NONE: return launch<CATOPT_EPI_NONE>(A, ldx, B, ldw, b1, b2, C, ldy, (int)M, (int)N, (int)K, batch, sA, sB, sC, s);
    case CATOPT_EPI_BIAS: return launch<CATOPT_EPI_BIAS>(A, ldx, B, ldw, b1, b2, C, ldy, (int)M, (int)N, (int)K, batch, sA, sB, sC, s);
    case CATOPT_EPI_BIAS_ADD2: return launch<CATOPT_EPI_BIAS_ADD2>(A, ldx, B, ldw, b1, b2, C, ldy, (int)M, (int)N, (int)K, batch, sA, sB, sC, s);
    case CATOPT_EPI_SILU_MUL: return launch<CATOPT_EPI_SILU_MUL>(A, ldx, B, ldw, b1, b2, C, ldy, (int)M, (int)N, (int)K, batch, sA, sB, sC, s);
    case CATOPT_EPI_GLU: return launch<CATOPT_EPI_GLU>(A, ldx, B, ldw, b1, b2, C, ldy, (int)M, (int)N, (int)K, batch, sA, sB, sC, s);
    default: return CATOPT_E_INVAL;
  }
}

}  // namespace catopt
