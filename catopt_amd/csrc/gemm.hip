// GEMM entry points: catopt_hip_linear and catopt_hip_matmul.
//
// bf16 with K-contiguous, 16-byte aligned operands goes to the 256x256
// bf16 MFMA kernel (gemm_bf16.hip).  Everything else — fp32 (the weight
// chain of the linear-bias association form and its construction-time
// fold), transposed operands, unaligned views — runs here on a 64x64-tile
// kernel using the 32x32x2 fp32 MFMA, with operands staged through LDS in
// k-contiguous order whatever their global layout.  bf16 operands are
// widened to fp32 in LDS (the products are exact), so both paths
// accumulate in fp32.
#include "common.hpp"

namespace catopt {
bool gemm_bf16_nt_fast_ok(int64_t M, int64_t N, int64_t K, const void* x, int64_t ldx,
                          const void* w, int64_t ldw, const void* y, int64_t ldy);
int32_t gemm_bf16_nt_launch(int32_t epi, int64_t M, int64_t N, int64_t K, const void* x,
                            int64_t ldx, const void* w, int64_t ldw, const void* bias,
                            const void* bias2, void* y, int64_t ldy, int64_t batch,
                            int64_t strideA, int64_t strideB, int64_t strideC, hipStream_t s);

namespace {

constexpr int TM = 64, TN = 64, TK = 32, NTH = 256;

__device__ __forceinline__ f32x16 mfma32x32x2f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// C[b] = epi(op(A[b]) op(B[b])).  TA: A stored K x M.  TB: B stored N x K
// (the linear-weight layout) — TB=false means B stored K x N.
// Paired epilogues read B rows n and n + N (TB must be true).
template <typename T, bool TA, bool TB, int EPI>
__global__ __launch_bounds__(NTH) void gemm_generic(
    const T* __restrict__ A, int64_t lda, int64_t sA, const T* __restrict__ B, int64_t ldb,
    int64_t sB, const T* __restrict__ bias, const T* __restrict__ bias2, T* __restrict__ C,
    int64_t ldc, int64_t sC, int M, int N, int K) {
  constexpr bool PAIRED = (EPI == CATOPT_EPI_SILU_MUL || EPI == CATOPT_EPI_GLU);
  constexpr int BROWS = PAIRED ? 2 * TN : TN;
  __shared__ float As[TM][TK + 1];
  __shared__ float Bs[BROWS][TK + 1];
  const int64_t bz = blockIdx.z;
  A += bz * sA;
  B += bz * sB;
  C += bz * sC;
  const int m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, g = lane >> 5;

  f32x16 acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc0[r] = acc1[r] = 0.f;

  for (int k0 = 0; k0 < K; k0 += TK) {
    // A tile -> As[m][k]
    for (int e = tid; e < TM * TK; e += NTH) {
      int m, k;
      if (TA) { k = e / TM; m = e % TM; } else { m = e / TK; k = e % TK; }
      const int gm = m0 + m, gk = k0 + k;
      float v = 0.f;
      if (gm < M && gk < K) v = load_f32(A, TA ? (int64_t)gk * lda + gm : (int64_t)gm * lda + gk);
      As[m][k] = v;
    }
    // B tile -> Bs[n][k]
    for (int e = tid; e < BROWS * TK; e += NTH) {
      int n, k;
      if (TB) { n = e / TK; k = e % TK; } else { k = e / BROWS; n = e % BROWS; }
      int gn;
      bool ok;
      if (PAIRED) {
        const int half = n / TN, nn = n % TN;
        ok = n0 + nn < N;
        gn = n0 + nn + half * N;
      } else {
        gn = n0 + n;
        ok = gn < N;
      }
      const int gk = k0 + k;
      float v = 0.f;
      if (ok && gk < K) v = load_f32(B, TB ? (int64_t)gn * ldb + gk : (int64_t)gk * ldb + gn);
      Bs[n][k] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < TK; kk += 2) {
      const float a = As[wm * 32 + l32][kk + g];
      const float b0 = Bs[wn * 32 + l32][kk + g];
      acc0 = mfma32x32x2f32(a, b0, acc0);
      if (PAIRED) {
        const float b1 = Bs[TN + wn * 32 + l32][kk + g];
        acc1 = mfma32x32x2f32(a, b1, acc1);
      }
    }
    __syncthreads();
  }

  const int n = n0 + wn * 32 + l32;
  if (n >= N) return;
  float badd = 0.f, badd2 = 0.f;
  if (EPI == CATOPT_EPI_BIAS || EPI == CATOPT_EPI_BIAS_ADD2) badd = load_f32(bias, n);
  if (EPI == CATOPT_EPI_BIAS_ADD2) badd2 = load_f32(bias2, n);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + wm * 32 + acc_row(r, g);
    if (m >= M) continue;
    float o;
    if (EPI == CATOPT_EPI_SILU_MUL) o = silu_f(acc0[r]) * acc1[r];
    else if (EPI == CATOPT_EPI_GLU) o = acc0[r] * sigmoid_f(acc1[r]);
    else o = (acc0[r] + badd) + badd2;
    store_f32(C, (int64_t)m * ldc + n, o);
  }
}

// ---------------------------------------------------------------- skinny fp32
// fp32 C[M, N] = epi(A[M, K] · W[N, K]ᵀ) for few rows (the folded weight
// chain: one 64 x 512 x 512 GEMM that the 64x64 tiles above spread over only
// 8 workgroups).  One workgroup per 16x16 output tile; its 4 waves split K
// into quarters and reduce the four 16x16 partials through LDS in a fixed
// order (deterministic).  Each lane stores its 4 accumulators with one
// 16-byte write at 16 l (consecutive lanes on consecutive chunks) and the
// reduction reads them back with consecutive lanes on consecutive words, so
// neither side has bank conflicts.  16x16x4 fp32 MFMA: lane l
// supplies A row l%16 and W row l%16 at k-group l/16; accumulator register
// r of lane l is output (4*(l/16) + r, l%16).  The k index of the MFMA is
// only a summation order, so each lane loads 4 consecutive k with one
// 16-byte load and feeds them to 4 consecutive MFMA steps (the same
// permutation on both operands).
#ifndef CATOPT_SK_CHUNK
#define CATOPT_SK_CHUNK 64
#endif
constexpr int SK_CHUNK = CATOPT_SK_CHUNK;  // k per wave per pass (one load round trip)
constexpr int SK_STEPS = SK_CHUNK / 16;    // 16-k steps per pass: 4 per lane group each

__device__ __forceinline__ f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_f32_skinny(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ W, int64_t ldw,
    const float* __restrict__ bias, const float* __restrict__ bias2, float* __restrict__ C,
    int64_t ldc, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) float part[4][64][4];  // [wave][lane][accumulator]
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, kq = lane >> 4;
  const int am = min(m0 + r16, M - 1), wn = min(n0 + r16, N - 1);  // clamped rows are never stored
  const float* arow = A + (int64_t)am * lda;
  const float* wrow = W + (int64_t)wn * ldw;
  const int kper = ((K + 4 * SK_CHUNK - 1) / (4 * SK_CHUNK)) * SK_CHUNK;  // k per wave, multiple of SK_CHUNK
  const int kbeg = wave * kper, kend = min(K, kbeg + kper);
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int kb = kbeg; kb < kend; kb += SK_CHUNK) {
    f32x4 av[SK_STEPS], bv[SK_STEPS];
#pragma unroll
    for (int s = 0; s < SK_STEPS; ++s) {
      const int k = kb + 16 * s + 4 * kq;  // K % 4 == 0: a group is wholly in or out
      const bool ok = k < kend;
      av[s] = ok ? *reinterpret_cast<const f32x4*>(arow + k) : f32x4{0.f, 0.f, 0.f, 0.f};
      bv[s] = ok ? *reinterpret_cast<const f32x4*>(wrow + k) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int s = 0; s < SK_STEPS; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = mfma16x16x4f32(av[s][e], bv[s][e], acc);
  }
  // lane l = 16 kq + r16 holds rows 4 kq .. 4 kq + 3 of column r16
  *reinterpret_cast<f32x4*>(&part[wave][lane][0]) = acc;
  __syncthreads();
  // lane t of wave w sums output (4 w + t % 4, t / 4), which every wave's
  // lane 16 w + t / 4 holds in accumulator t % 4: word 64 w + t of each block
  const int i = 4 * wave + (lane & 3), j = lane >> 2;
  const int src = 16 * wave + j;
  const int m = m0 + i, n = n0 + j;
  if (m >= M || n >= N) return;
  float o = ((part[0][src][i & 3] + part[1][src][i & 3]) + part[2][src][i & 3]) + part[3][src][i & 3];
  if (EPI == CATOPT_EPI_BIAS || EPI == CATOPT_EPI_BIAS_ADD2) o += bias[n];
  if (EPI == CATOPT_EPI_BIAS_ADD2) o += bias2[n];
  C[(int64_t)m * ldc + n] = o;
}

bool skinny_ok(int64_t M, int64_t N, int64_t K, const void* x, int64_t ldx, const void* w,
               int64_t ldw) {
  const int64_t tiles64 = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
  return tiles64 < 256 && M <= 1024 && K % 4 == 0 && ldx % 4 == 0 && ldw % 4 == 0 &&
         aligned16(x) && aligned16(w) && (N + 15) / 16 <= 0x7fffffffLL && (M + 15) / 16 <= 65535;
}

int32_t launch_skinny(int32_t epi, const float* A, int64_t lda, const float* W, int64_t ldw,
                      const float* bias, const float* bias2, float* C, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, hipStream_t s) {
  const dim3 grid((uint32_t)((N + 15) / 16), (uint32_t)((M + 15) / 16));
  switch (epi) {
    case CATOPT_EPI_NONE:
      gemm_f32_skinny<CATOPT_EPI_NONE><<<grid, 256, 0, s>>>(A, lda, W, ldw, bias, bias2, C, ldc, (int)M, (int)N, (int)K);
      break;
    case CATOPT_EPI_BIAS:
      gemm_f32_skinny<CATOPT_EPI_BIAS><<<grid, 256, 0, s>>>(A, lda, W, ldw, bias, bias2, C, ldc, (int)M, (int)N, (int)K);
      break;
    case CATOPT_EPI_BIAS_ADD2:
      gemm_f32_skinny<CATOPT_EPI_BIAS_ADD2><<<grid, 256, 0, s>>>(A, lda, W, ldw, bias, bias2, C, ldc, (int)M, (int)N, (int)K);
      break;
    default:
      return CATOPT_E_INVAL;
  }
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

template <typename T, bool TA, bool TB, int EPI>
int32_t launch_generic(const void* A, int64_t lda, int64_t sA, const void* B, int64_t ldb,
                       int64_t sB, const void* bias, const void* bias2, void* C, int64_t ldc,
                       int64_t sC, int64_t batch, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  const int64_t gx = (N + TN - 1) / TN, gy = (M + TM - 1) / TM;
  if (gx > 0x7fffffff || gy > 65535 || batch > 65535) return CATOPT_E_UNSUPPORTED;
  gemm_generic<T, TA, TB, EPI><<<dim3((uint32_t)gx, (uint32_t)gy, (uint32_t)batch), dim3(NTH), 0, s>>>(
      static_cast<const T*>(A), lda, sA, static_cast<const T*>(B), ldb, sB,
      static_cast<const T*>(bias), static_cast<const T*>(bias2), static_cast<T*>(C), ldc, sC,
      (int)M, (int)N, (int)K);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

template <typename T, bool TA, bool TB>
int32_t dispatch_epi(int32_t epi, const void* A, int64_t lda, int64_t sA, const void* B,
                     int64_t ldb, int64_t sB, const void* bias, const void* bias2, void* C,
                     int64_t ldc, int64_t sC, int64_t batch, int64_t M, int64_t N, int64_t K,
                     hipStream_t s) {
  switch (epi) {
    case CATOPT_EPI_NONE:
      return launch_generic<T, TA, TB, CATOPT_EPI_NONE>(A, lda, sA, B, ldb, sB, bias, bias2, C, ldc, sC, batch, M, N, K, s);
    case CATOPT_EPI_BIAS:
      return launch_generic<T, TA, TB, CATOPT_EPI_BIAS>(A, lda, sA, B, ldb, sB, bias, bias2, C, ldc, sC, batch, M, N, K, s);
    case CATOPT_EPI_BIAS_ADD2:
      return launch_generic<T, TA, TB, CATOPT_EPI_BIAS_ADD2>(A, lda, sA, B, ldb, sB, bias, bias2, C, ldc, sC, batch, M, N, K, s);
    default:
      return CATOPT_E_INVAL;
  }
}

template <typename T>
int32_t dispatch_paired(int32_t epi, const void* A, int64_t lda, const void* B, int64_t ldb,
                        void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  if (epi == CATOPT_EPI_SILU_MUL)
    return launch_generic<T, false, true, CATOPT_EPI_SILU_MUL>(A, lda, 0, B, ldb, 0, nullptr, nullptr, C, ldc, 0, 1, M, N, K, s);
  return launch_generic<T, false, true, CATOPT_EPI_GLU>(A, lda, 0, B, ldb, 0, nullptr, nullptr, C, ldc, 0, 1, M, N, K, s);
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int32_t catopt_hip_linear(int32_t dtype, int64_t M, int64_t N, int64_t K,
                                     const void* x, int64_t ldx, const void* w, int64_t ldw,
                                     const void* bias, const void* bias2, int32_t epilogue,
                                     void* y, int64_t ldy, void* stream) {
  if (M < 0 || N < 0 || K < 0) return CATOPT_E_INVAL;
  if (epilogue < CATOPT_EPI_NONE || epilogue > CATOPT_EPI_GLU) return CATOPT_E_INVAL;
  if (dtype != CATOPT_F32 && dtype != CATOPT_BF16) return CATOPT_E_UNSUPPORTED;
  if (M == 0 || N == 0) return CATOPT_OK;
  if (K == 0) return CATOPT_E_UNSUPPORTED;  // an empty contraction: leave to the caller
  if (!x || !w || !y || ldx < K || ldw < K || ldy < N) return CATOPT_E_INVAL;
  const bool paired = epilogue == CATOPT_EPI_SILU_MUL || epilogue == CATOPT_EPI_GLU;
  if ((epilogue == CATOPT_EPI_BIAS || epilogue == CATOPT_EPI_BIAS_ADD2) && !bias) return CATOPT_E_INVAL;
  if (epilogue == CATOPT_EPI_BIAS_ADD2 && !bias2) return CATOPT_E_INVAL;
  if (M > 0x7fffffffLL || N > 0x3fffffffLL || K > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == CATOPT_BF16 && gemm_bf16_nt_fast_ok(M, N, K, x, ldx, w, ldw, y, ldy))
    return gemm_bf16_nt_launch(epilogue, M, N, K, x, ldx, w, ldw, bias, bias2, y, ldy, 1, 0, 0, 0, s);
  if (dtype == CATOPT_F32 && !paired && skinny_ok(M, N, K, x, ldx, w, ldw))
    return launch_skinny(epilogue, static_cast<const float*>(x), ldx, static_cast<const float*>(w), ldw,
                         static_cast<const float*>(bias), static_cast<const float*>(bias2),
                         static_cast<float*>(y), ldy, M, N, K, s);
  if (paired) {
    return dtype == CATOPT_BF16 ? dispatch_paired<uint16_t>(epilogue, x, ldx, w, ldw, y, ldy, M, N, K, s)
                                : dispatch_paired<float>(epilogue, x, ldx, w, ldw, y, ldy, M, N, K, s);
  }
  return dtype == CATOPT_BF16
             ? dispatch_epi<uint16_t, false, true>(epilogue, x, ldx, 0, w, ldw, 0, bias, bias2, y, ldy, 0, 1, M, N, K, s)
             : dispatch_epi<float, false, true>(epilogue, x, ldx, 0, w, ldw, 0, bias, bias2, y, ldy, 0, 1, M, N, K, s);
}

extern "C" int32_t catopt_hip_matmul(int32_t dtype, int64_t batch, int64_t M, int64_t N,
                                     int64_t K, const void* A, int64_t lda, int64_t strideA,
                                     int32_t transA, const void* B, int64_t ldb, int64_t strideB,
                                     int32_t transB, void* C, int64_t ldc, int64_t strideC,
                                     void* stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0) return CATOPT_E_INVAL;
  if (dtype != CATOPT_F32 && dtype != CATOPT_BF16) return CATOPT_E_UNSUPPORTED;
  if (batch == 0 || M == 0 || N == 0) return CATOPT_OK;
  if (K == 0) return CATOPT_E_UNSUPPORTED;
  if (!A || !B || !C || ldc < N) return CATOPT_E_INVAL;
  if ((transA ? lda < M : lda < K) || (transB ? ldb < K : ldb < N)) return CATOPT_E_INVAL;
  if (M > 0x7fffffffLL || N > 0x3fffffffLL || K > 0x7fffffffLL) return CATOPT_E_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool strides_ok = strideA % 8 == 0 && strideB % 8 == 0;
  if (dtype == CATOPT_BF16 && !transA && transB && strides_ok &&
      gemm_bf16_nt_fast_ok(M, N, K, A, lda, B, ldb, C, ldc))
    return gemm_bf16_nt_launch(CATOPT_EPI_NONE, M, N, K, A, lda, B, ldb, nullptr, nullptr, C, ldc,
                               batch, strideA, strideB, strideC, s);
#define CATOPT_MM(T)                                                                                          \
  if (!transA && !transB) return dispatch_epi<T, false, false>(0, A, lda, strideA, B, ldb, strideB, nullptr, nullptr, C, ldc, strideC, batch, M, N, K, s); \
  if (!transA && transB) return dispatch_epi<T, false, true>(0, A, lda, strideA, B, ldb, strideB, nullptr, nullptr, C, ldc, strideC, batch, M, N, K, s);   \
  if (transA && !transB) return dispatch_epi<T, true, false>(0, A, lda, strideA, B, ldb, strideB, nullptr, nullptr, C, ldc, strideC, batch, M, N, K, s);   \
  return dispatch_epi<T, true, true>(0, A, lda, strideA, B, ldb, strideB, nullptr, nullptr, C, ldc, strideC, batch, M, N, K, s);
  if (dtype == CATOPT_BF16) {
    CATOPT_MM(uint16_t)
  }
  CATOPT_MM(float)
#undef CATOPT_MM
}
