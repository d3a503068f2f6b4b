// Diagonal affine scans on gfx950 (fp32).
//
// Both kernels are HBM-streaming: every lane owns state elements and walks
// the time axis.  The loads of a block of U steps are issued one block ahead
// of the arithmetic (register double buffering), so each wave keeps
// U x 16 B x 64 lanes of reads in flight while it computes.
//
// Schedules (the int64 chunk table chunk_starts[0..n] cuts [0, T)):
//   STREAM  — one pass; a lane walks the chunks in table order.  HBM-optimal
//             (a is read once) and used whenever the lanes fill the GPU.
//   CHUNKED — three launches: (1) every chunk composes its own map
//             (P = prod a, H = local state from 0), chunk-parallel;
//             (2) per lane, fold the carries over chunks in table order,
//             leaving the carry-in of each chunk in the workspace;
//             (3) every chunk re-runs from its carry-in and emits outputs.
//             This is the two-level blocked scan of the reference's
//             all-prefix path; it trades a second read of the inputs for
//             chunk-level parallelism when B*D*N alone cannot fill the GPU.
#include <mutex>

#include "common.hpp"

namespace catopt {
namespace {

constexpr int kThreads = 256;

// Chunk bounds clamped to [0, T]: a malformed table can only shorten the
// walk, never index outside the inputs (the host validates the table too).
__device__ __forceinline__ int64_t cclamp(int64_t v, int64_t T) { return v < 0 ? 0 : (v > T ? T : v); }

// ---------------------------------------------------------------- affd scan
// h_t = a_t * h_{t-1} + u_t over [t0, t1) for lane s.
__device__ __forceinline__ float affd_run(const float* __restrict__ a, int64_t lda,
                                          const float* __restrict__ u, int64_t ldu,
                                          float* __restrict__ states, int64_t S, int64_t s,
                                          int64_t t0, int64_t t1, float h, float* prod) {
  constexpr int U = 8;
  float p = 1.f;
  int64_t t = t0;
  for (; t + U <= t1; t += U) {
    float av[U], uv[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      av[i] = a[(t + i) * lda + s];
      uv[i] = u[(t + i) * ldu + s];
    }
#pragma unroll
    for (int i = 0; i < U; ++i) {
      h = av[i] * h + uv[i];
      p *= av[i];
      if (states) states[(t + i) * S + s] = h;
    }
  }
  for (; t < t1; ++t) {
    const float av = a[t * lda + s];
    h = av * h + u[t * ldu + s];
    p *= av;
    if (states) states[t * S + s] = h;
  }
  if (prod) *prod = p;
  return h;
}

__global__ __launch_bounds__(kThreads) void affd_stream(
    const float* __restrict__ a, int64_t lda, const float* __restrict__ u, int64_t ldu,
    const float* __restrict__ h0, const int64_t* __restrict__ cs, int64_t nc, int64_t T, int64_t S,
    float* __restrict__ states, float* __restrict__ hf) {
  const int64_t s = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (s >= S) return;
  float h = h0 ? h0[s] : 0.f;
  for (int64_t c = 0; c < nc; ++c)
    h = affd_run(a, lda, u, ldu, states, S, s, cclamp(cs[c], T), cclamp(cs[c + 1], T), h, nullptr);
  if (hf) hf[s] = h;
}

// Phase 1: ws_p[c, s] = prod of a over chunk c; ws_h[c, s] = chunk-local state.
__global__ __launch_bounds__(kThreads) void affd_chunk_local(
    const float* __restrict__ a, int64_t lda, const float* __restrict__ u, int64_t ldu,
    const int64_t* __restrict__ cs, int64_t T, int64_t S, float* __restrict__ ws_p,
    float* __restrict__ ws_h) {
  const int64_t s = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t c = blockIdx.y;
  if (s >= S) return;
  float p;
  const float h = affd_run(a, lda, u, ldu, nullptr, S, s, cclamp(cs[c], T), cclamp(cs[c + 1], T), 0.f, &p);
  ws_p[c * S + s] = p;
  ws_h[c * S + s] = h;
}

// Phase 2: carry fold; ws_h[c, s] becomes the state entering chunk c.
__global__ __launch_bounds__(kThreads) void scan_carry(const float* __restrict__ h0, int64_t nc,
                                                       int64_t S, const float* __restrict__ ws_p,
                                                       float* __restrict__ ws_h,
                                                       float* __restrict__ hf) {
  const int64_t s = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (s >= S) return;
  float cin = h0 ? h0[s] : 0.f;
  // the chunk summaries do not depend on the carry: load a batch of them
  // before the batch's stores (which the compiler cannot reorder across
  // ws_h's loads), so a batch costs one memory latency, not one per chunk
  constexpr int kBatch = 16;
  for (int64_t c0 = 0; c0 < nc; c0 += kBatch) {
    const int n = (int)(nc - c0 < kBatch ? nc - c0 : kBatch);
    float p[kBatch], h[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (i < n) {
        p[i] = ws_p[(c0 + i) * S + s];
        h[i] = ws_h[(c0 + i) * S + s];
      }
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (i < n) {
        ws_h[(c0 + i) * S + s] = cin;
        cin = p[i] * cin + h[i];
      }
  }
  if (hf) hf[s] = cin;
}

// Phase 3: re-run each chunk from its carry-in, writing the prefix states.
__global__ __launch_bounds__(kThreads) void affd_chunk_apply(
    const float* __restrict__ a, int64_t lda, const float* __restrict__ u, int64_t ldu,
    const int64_t* __restrict__ cs, int64_t T, int64_t S, const float* __restrict__ ws_h,
    float* __restrict__ states) {
  const int64_t s = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t c = blockIdx.y;
  if (s >= S) return;
  affd_run(a, lda, u, ldu, states, S, s, cclamp(cs[c], T), cclamp(cs[c + 1], T), ws_h[c * S + s], nullptr);
}

// ---------------------------------------------------------------- SSM scan
// Thread layout: TPD = N/4 threads per channel d, each owning 4 consecutive
// state elements n (one 16-byte load of a per step); DPW = 256/TPD channels
// per workgroup; grid.y = batch.  y[b,t,d] is reduced across the TPD lanes
// of a channel with xor shuffles (DPP quad-perm / ds_swizzle patterns).
template <int N>
struct SsmLayout {
  static constexpr int TPD = N / 4;
  static constexpr int DPW = kThreads / TPD;
};

template <int N, bool APS>
struct SsmStep {
  f32x4 a;
  f32x4 bx;
  f32x4 c;
  float x;
};

template <int N, bool APS>
__device__ __forceinline__ void ssm_load(SsmStep<N, APS>& st, const float* __restrict__ a,
                                         const float* __restrict__ bx,
                                         const float* __restrict__ c,
                                         const float* __restrict__ x, int64_t b, int64_t t,
                                         int64_t T, int64_t D, int64_t d, int n0) {
  const int64_t bt = b * T + t;
  if (APS) {
    st.a = *reinterpret_cast<const f32x4*>(a + (bt * D + d) * N + n0);
  } else {
    const float av = a[bt * D + d];
    st.a = f32x4{av, av, av, av};
  }
  st.bx = *reinterpret_cast<const f32x4*>(bx + bt * N + n0);
  st.c = *reinterpret_cast<const f32x4*>(c + bt * N + n0);
  st.x = x[bt * D + d];
}

template <int N>
__device__ __forceinline__ float lane_reduce(float p) {
#pragma unroll
  for (int o = 1; o < SsmLayout<N>::TPD; o <<= 1) p += __shfl_xor(p, o, 64);
  return p;
}

// Run steps [t0, t1) from state h; optionally emit y and the product of a.
template <int N, bool APS, bool EMIT>
__device__ __forceinline__ f32x4 ssm_run(const float* __restrict__ a,
                                         const float* __restrict__ bx,
                                         const float* __restrict__ c,
                                         const float* __restrict__ x, float* __restrict__ y,
                                         int64_t b, int64_t T, int64_t D, int64_t d, bool dok,
                                         int n0, int64_t t0, int64_t t1, f32x4 h, f32x4* prod) {
  constexpr int U = 8;
  const int64_t dd = dok ? d : 0;  // out-of-range channels shadow channel 0, never store
  f32x4 p = f32x4{1.f, 1.f, 1.f, 1.f};
  SsmStep<N, APS> cur[U], nxt[U];
  int64_t t = t0;
  if (t + U <= t1) {
#pragma unroll
    for (int i = 0; i < U; ++i) ssm_load(cur[i], a, bx, c, x, b, t + i, T, D, dd, n0);
  }
  for (; t + U <= t1; t += U) {
    const bool more = t + 2 * U <= t1;
    if (more) {
#pragma unroll
      for (int i = 0; i < U; ++i) ssm_load(nxt[i], a, bx, c, x, b, t + U + i, T, D, dd, n0);
    }
#pragma unroll
    for (int i = 0; i < U; ++i) {
      h = cur[i].a * h + cur[i].bx * cur[i].x;
      if (!EMIT) p *= cur[i].a;
      if (EMIT) {
        const f32x4 ch = cur[i].c * h;
        const float r = lane_reduce<N>(ch[0] + ch[1] + ch[2] + ch[3]);
        if (dok && n0 == 0) y[(b * T + t + i) * D + d] = r;
      }
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < U; ++i) cur[i] = nxt[i];
    }
  }
  for (; t < t1; ++t) {
    SsmStep<N, APS> st;
    ssm_load(st, a, bx, c, x, b, t, T, D, dd, n0);
    h = st.a * h + st.bx * st.x;
    if (!EMIT) p *= st.a;
    if (EMIT) {
      const f32x4 ch = st.c * h;
      const float r = lane_reduce<N>(ch[0] + ch[1] + ch[2] + ch[3]);
      if (dok && n0 == 0) y[(b * T + t) * D + d] = r;
    }
  }
  if (prod) *prod = p;
  return h;
}

template <int N>
struct SsmIdx {
  int64_t d;
  bool dok;
  int n0;
};

template <int N>
__device__ __forceinline__ SsmIdx<N> ssm_idx(int64_t D) {
  SsmIdx<N> r;
  const int tl = threadIdx.x;
  r.d = (int64_t)blockIdx.x * SsmLayout<N>::DPW + tl / SsmLayout<N>::TPD;
  r.dok = r.d < D;
  r.n0 = (tl % SsmLayout<N>::TPD) * 4;
  return r;
}

template <int N, bool APS>
__global__ __launch_bounds__(kThreads) void ssm_stream(
    const float* __restrict__ a, const float* __restrict__ bx, const float* __restrict__ c,
    const float* __restrict__ x, const float* __restrict__ h0, const int64_t* __restrict__ cs,
    int64_t nc, int64_t T, int64_t D, float* __restrict__ y, float* __restrict__ hf) {
  const SsmIdx<N> ix = ssm_idx<N>(D);
  const int64_t b = blockIdx.y;
  f32x4 h = f32x4{0.f, 0.f, 0.f, 0.f};
  const int64_t sidx = (b * D + ix.d) * N + ix.n0;
  if (h0 && ix.dok) h = *reinterpret_cast<const f32x4*>(h0 + sidx);
  for (int64_t k = 0; k < nc; ++k)
    h = ssm_run<N, APS, true>(a, bx, c, x, y, b, T, D, ix.d, ix.dok, ix.n0, cclamp(cs[k], T),
                              cclamp(cs[k + 1], T), h, nullptr);
  if (hf && ix.dok) *reinterpret_cast<f32x4*>(hf + sidx) = h;
}

template <int N, bool APS>
__global__ __launch_bounds__(kThreads) void ssm_chunk_local(
    const float* __restrict__ a, const float* __restrict__ bx, const float* __restrict__ c,
    const float* __restrict__ x, const int64_t* __restrict__ cs, int64_t T, int64_t D,
    int64_t S, float* __restrict__ ws_p, float* __restrict__ ws_h) {
  const SsmIdx<N> ix = ssm_idx<N>(D);
  const int64_t b = blockIdx.y, k = blockIdx.z;
  f32x4 p;
  const f32x4 h = ssm_run<N, APS, false>(a, bx, c, x, nullptr, b, T, D, ix.d, ix.dok, ix.n0,
                                         cclamp(cs[k], T), cclamp(cs[k + 1], T),
                                         f32x4{0.f, 0.f, 0.f, 0.f}, &p);
  if (!ix.dok) return;
  const int64_t sidx = (b * D + ix.d) * N + ix.n0;
  *reinterpret_cast<f32x4*>(ws_p + k * S + sidx) = p;
  *reinterpret_cast<f32x4*>(ws_h + k * S + sidx) = h;
}

template <int N, bool APS>
__global__ __launch_bounds__(kThreads) void ssm_chunk_apply(
    const float* __restrict__ a, const float* __restrict__ bx, const float* __restrict__ c,
    const float* __restrict__ x, const int64_t* __restrict__ cs, int64_t T, int64_t D,
    int64_t S, const float* __restrict__ ws_h, float* __restrict__ y) {
  const SsmIdx<N> ix = ssm_idx<N>(D);
  const int64_t b = blockIdx.y, k = blockIdx.z;
  const int64_t sidx = (b * D + (ix.dok ? ix.d : 0)) * N + ix.n0;
  const f32x4 h = *reinterpret_cast<const f32x4*>(ws_h + k * S + sidx);
  ssm_run<N, APS, true>(a, bx, c, x, y, b, T, D, ix.d, ix.dok, ix.n0, cclamp(cs[k], T),
                        cclamp(cs[k + 1], T), h, nullptr);
}

// ----------------------------------------------------- LDS-staged streaming
// The streaming schedule for a per-state a (B, T, D, N), fed through LDS:
// a workgroup owns DPW channels x N states (one 4 KB slice of a per step)
// and streams U-step stages of a, b, c and x into LDS with direct
// global->LDS loads (no registers held while the loads are in flight), two
// stages deep: the loads of stage s+1 are issued before the arithmetic of
// stage s and waited for after it, one barrier per stage.  Each workgroup
// thus keeps U x ~4.4 KB of reads in flight, two workgroups per CU, which is
// what HBM's bandwidth-latency product asks of 256 CUs.  The chunk table
// tiles [0, T) in order, so one pass over t = 0 .. T-1 is that walk.
constexpr int SU = 8;  // steps per LDS stage

template <int N>
struct SsmLds {
  static constexpr int TPD = N / 4, DPW = kThreads / TPD;
  static constexpr int A_BYTES = SU * DPW * N * 4;   // SU x 4 KB
  static constexpr int X_BYTES = SU * DPW * 4;
  static constexpr int V_BYTES = SU * N * 4;         // b or c
  static constexpr int STAGE = A_BYTES + X_BYTES + 2 * V_BYTES;
  static constexpr int BYTES = 2 * STAGE;
  static constexpr int X_SLOTS = SU * DPW;           // 4-byte slots
  static constexpr int V_SLOTS = SU * N;
};

typedef __attribute__((address_space(3))) void* lds_vptr;

template <int N>
__global__ __launch_bounds__(kThreads, 2) void ssm_stream_lds(
    const float* __restrict__ a, const float* __restrict__ bx, const float* __restrict__ c,
    const float* __restrict__ x, const float* __restrict__ h0, int64_t T, int64_t D,
    float* __restrict__ y, float* __restrict__ hf) {
  using L = SsmLds<N>;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t b = blockIdx.y;
  const int64_t d0 = (int64_t)blockIdx.x * L::DPW;
  const int ch = tid / L::TPD, n0 = (tid % L::TPD) * 4;
  const int64_t d = d0 + ch;
  const bool dok = d < D;
  // a slot of this thread: channel d (clamped to a valid one), states n0..n0+3
  const int64_t a_lane = (((dok ? d : D - 1) * N) + n0);
  const int64_t nst = (T + SU - 1) / SU;

  auto issue = [&](int64_t st, int stage) {
    char* base = lds + stage * L::STAGE;
    const int64_t t0 = st * SU;
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int64_t t = t0 + u < T ? t0 + u : T - 1;
      const float* src = a + ((b * T + t) * D) * N + a_lane;
      __builtin_amdgcn_global_load_lds(src, (lds_vptr)(base + u * (L::DPW * N * 4) + wave * 1024), 16, 0, 0);
    }
    char* xb = base + L::A_BYTES;
#pragma unroll
    for (int i = 0; i < (L::X_SLOTS + kThreads - 1) / kThreads; ++i) {
      const int s = i * kThreads + tid;
      if (i * kThreads + wave * 64 < L::X_SLOTS) {  // whole waves: DPW*SU is a multiple of 64
        const int u = s / L::DPW, cc = s % L::DPW;
        const int64_t t = t0 + u < T ? t0 + u : T - 1;
        const int64_t dd = d0 + cc < D ? d0 + cc : D - 1;
        __builtin_amdgcn_global_load_lds(x + (b * T + t) * D + dd,
                                         (lds_vptr)(xb + (i * kThreads + wave * 64) * 4), 4, 0, 0);
      }
    }
    char* vb = xb + L::X_BYTES;
#pragma unroll
    for (int i = 0; i < (L::V_SLOTS + kThreads - 1) / kThreads; ++i) {
      const int s = i * kThreads + tid;
      if (s < L::V_SLOTS) {
        const int u = s / N, n = s % N;
        const int64_t t = t0 + u < T ? t0 + u : T - 1;
        const int64_t off = (b * T + t) * N + n;
        const int lbase = (i * kThreads + wave * 64) * 4;
        __builtin_amdgcn_global_load_lds(bx + off, (lds_vptr)(vb + lbase), 4, 0, 0);
        __builtin_amdgcn_global_load_lds(c + off, (lds_vptr)(vb + L::V_BYTES + lbase), 4, 0, 0);
      }
    }
  };

  f32x4 h = f32x4{0.f, 0.f, 0.f, 0.f};
  const int64_t sidx = (b * D + (dok ? d : 0)) * N + n0;
  if (h0 && dok) h = *reinterpret_cast<const f32x4*>(h0 + sidx);
  if (nst > 0) {
    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  for (int64_t st = 0; st < nst; ++st) {
    const int cur = (int)(st & 1);
    if (st + 1 < nst) issue(st + 1, cur ^ 1);
    const char* base = lds + cur * L::STAGE;
    const char* xb = base + L::A_BYTES;
    const char* vb = xb + L::X_BYTES;
    const int64_t t0 = st * SU;
    const int un = T - t0 < SU ? (int)(T - t0) : SU;
    for (int u = 0; u < un; ++u) {
      const f32x4 av = *reinterpret_cast<const f32x4*>(base + u * (L::DPW * N * 4) + tid * 16);
      const f32x4 bv = *reinterpret_cast<const f32x4*>(vb + (u * N + n0) * 4);
      const f32x4 cv = *reinterpret_cast<const f32x4*>(vb + L::V_BYTES + (u * N + n0) * 4);
      const float xv = *reinterpret_cast<const float*>(xb + (u * L::DPW + ch) * 4);
      h = av * h + bv * xv;
      const f32x4 chv = cv * h;
      const float r = lane_reduce<N>(chv[0] + chv[1] + chv[2] + chv[3]);
      if (dok && n0 == 0) y[(b * T + t0 + u) * D + d] = r;
    }
    if (st + 1 < nst) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }
  if (hf && dok) *reinterpret_cast<f32x4*>(hf + sidx) = h;
}

// --------------------------------------------------- register-staged streaming
// The streaming schedule for a per-state a (N = 16) with a held in registers:
// each thread's 16-byte slices of a for RSU steps go straight into one of
// two register sets while the other set's steps run; the small x, b and c
// streams go through LDS (one copy per workgroup) by direct loads issued
// before a's, and y leaves through LDS as whole rows.  Every wave issues the
// same memory operations in every stage with no branch around them, so the
// waits the compiler derives for a are exact, and the wait at the end of a
// stage leaves the RSU newest loads (the next stage's a) in flight across
// the barrier: two stages of a (2 x RSU x 4 KB per workgroup) stay in
// flight and no stage drains the memory pipeline.  On gfx9 stores count in
// vmcnt too, which is why y is not stored step by step under a lane mask.
// y's stores are non-temporal (written once, never read back here): 1.5%
// faster at C5's shape than plain stores.  What y costs beyond that is
// HBM's turnaround between reads and writes; a plain streaming kernel with
// the same 16:1 read/write mix pays it as well.  Steps past the last whole
// stage run unpipelined.  (The LDS-staged kernel above waits for all its
// loads at every stage, which measured 5-14% slower at C5's shape.)
#ifndef CATOPT_SSM_RSU
#define CATOPT_SSM_RSU 8
#endif
constexpr int RSU = CATOPT_SSM_RSU;  // steps per stage of the register-staged scan

template <int N>
struct SsmSmall {
  static constexpr int TPD = N / 4, DPW = kThreads / TPD;
  static constexpr int X_BYTES = RSU * DPW * 4;
  static constexpr int V_BYTES = RSU * N * 4;   // b or c
  static constexpr int STAGE = X_BYTES + 2 * V_BYTES;
  static constexpr int Y_BYTES = RSU * DPW * 4;
  static constexpr int BYTES = 2 * STAGE + 2 * Y_BYTES;
  static constexpr int XPT = RSU * DPW / kThreads;         // x loads (and y stores) per thread
  static constexpr int VPT = 2 * RSU * N / kThreads;       // b and c loads per thread
  static_assert(RSU * DPW % kThreads == 0 && 2 * RSU * N % kThreads == 0, "whole waves per small stream");
  static_assert(RSU * N % 64 == 0, "b and c slots in whole waves");
};

template <int N>
__global__ __launch_bounds__(kThreads, 2) void ssm_stream_reg(
    const float* __restrict__ a, const float* __restrict__ bx, const float* __restrict__ c,
    const float* __restrict__ x, const float* __restrict__ h0, int64_t T, int64_t D,
    float* __restrict__ y, float* __restrict__ hf) {
  using L = SsmSmall<N>;
  __shared__ __attribute__((aligned(16))) char lds[L::BYTES];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t b = blockIdx.y;
  const int64_t d0 = (int64_t)blockIdx.x * L::DPW;
  const int ch = tid / L::TPD, n0 = (tid % L::TPD) * 4;
  const int64_t d = d0 + ch;
  const bool dok = d < D;
  const int64_t a_lane = (((dok ? d : D - 1) * N) + n0);
  const int64_t nfull = T / RSU;
  // this thread's small-stream slots: x (u, channel) for two slots; b (waves
  // 0, 1) or c (waves 2, 3) for one (u, n) slot, clamped to valid rows
  int xu[L::XPT], xc[L::XPT];
#pragma unroll
  for (int i = 0; i < L::XPT; ++i) {
    const int s = i * kThreads + tid;
    xu[i] = s / L::DPW;
    xc[i] = (int)(d0 + s % L::DPW < D ? s % L::DPW : D - 1 - d0);
  }

  const uint32_t lds0 = lds_u32(lds);
  auto issue_small = [&](int64_t st, int stage) {
    const uint32_t xb = lds0 + stage * L::STAGE;
    const int64_t t0 = st * RSU;
#pragma unroll
    for (int i = 0; i < L::XPT; ++i)
      dma4(x + (b * T + t0 + xu[i]) * D + d0 + xc[i], xb + (i * kThreads + wave * 64) * 4);
    // b then c, one 4-byte slot per lane: slots [0, RSU*N) of b, then of c
#pragma unroll
    for (int i = 0; i < L::VPT; ++i) {
      const int s = i * kThreads + tid;
      const bool is_c = s >= RSU * N;              // wave-uniform: RSU*N is a multiple of 64
      const int vs = is_c ? s - RSU * N : s;
      dma4((is_c ? c : bx) + (b * T + t0 + vs / N) * N + vs % N,
           __builtin_amdgcn_readfirstlane(xb + L::X_BYTES + (is_c ? L::V_BYTES : 0) + (vs & ~63) * 4));
    }
  };
  auto load_a = [&](int64_t st, f32x4* ra) {
    const int64_t t0 = st * RSU;
#pragma unroll
    for (int u = 0; u < RSU; ++u)
      ra[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a + ((b * T + t0 + u) * D) * N + a_lane));
  };

  f32x4 h = f32x4{0.f, 0.f, 0.f, 0.f};
  const int64_t sidx = (b * D + (dok ? d : 0)) * N + n0;
  if (h0 && dok) h = *reinterpret_cast<const f32x4*>(h0 + sidx);
  auto compute = [&](int stage, const f32x4* ra, char* yb) {
    const char* xb = lds + stage * L::STAGE;
    const char* vb = xb + L::X_BYTES;
#pragma unroll
    for (int u = 0; u < RSU; ++u) {
      const f32x4 bv = *reinterpret_cast<const f32x4*>(vb + (u * N + n0) * 4);
      const f32x4 cv = *reinterpret_cast<const f32x4*>(vb + L::V_BYTES + (u * N + n0) * 4);
      const float xv = *reinterpret_cast<const float*>(xb + (u * L::DPW + ch) * 4);
      h = ra[u] * h + bv * xv;
      const f32x4 chv = cv * h;
      const float r = lane_reduce<N>(chv[0] + chv[1] + chv[2] + chv[3]);
      if (n0 == 0) *reinterpret_cast<float*>(yb + (u * L::DPW + ch) * 4) = r;
    }
  };
  // y rows of a stage from LDS: row u, channels d0 .. d0 + DPW - 1
  auto store_y = [&](int64_t st, const char* yb) {
#pragma unroll
    for (int i = 0; i < L::XPT; ++i) {
      // a channel past D (last, partial workgroup) writes channel D - 1's
      // value to it again: no lane mask around the store
      const int u = (i * kThreads + tid) / L::DPW;
      const int cc = xc[i];  // the clamped channel of slot i
      __builtin_nontemporal_store(*reinterpret_cast<const float*>(yb + (u * L::DPW + cc) * 4),
                                  y + (b * T + st * RSU + u) * D + d0 + cc);
    }
  };
  char* ybuf0 = lds + 2 * L::STAGE;
  char* ybuf1 = ybuf0 + L::Y_BYTES;
  auto step = [&](int64_t st, int buf, f32x4* cur, f32x4* nxt) {
    const int64_t sn = st + 1 < nfull ? st + 1 : nfull - 1;  // the last stage reloads itself
    issue_small(sn, buf ^ 1);
    load_a(sn, nxt);
    char* yb = buf ? ybuf1 : ybuf0;
    compute(buf, cur, yb);
    __builtin_amdgcn_s_waitcnt((RSU & 15) | (7 << 4) | ((RSU >> 4) << 14));  // vmcnt <= RSU, lgkmcnt 0
    __syncthreads();
    store_y(st, yb);
  };
  f32x4 ra0[RSU], ra1[RSU];
  if (nfull > 0) {
    issue_small(0, 0);
    load_a(0, ra0);
    __builtin_amdgcn_s_waitcnt((RSU & 15) | (7 << 4) | ((RSU >> 4) << 14));
    __syncthreads();
    for (int64_t st = 0; st < nfull; st += 2) {
      step(st, 0, ra0, ra1);
      if (st + 1 < nfull) step(st + 1, 1, ra1, ra0);
    }
  }
  // steps past the last whole stage
  for (int64_t t = nfull * RSU; t < T; ++t) {
    SsmStep<N, true> sp;
    ssm_load(sp, a, bx, c, x, b, t, T, D, dok ? d : 0, n0);
    h = sp.a * h + sp.bx * sp.x;
    const f32x4 chv = sp.c * h;
    const float r = lane_reduce<N>(chv[0] + chv[1] + chv[2] + chv[3]);
    if (dok && n0 == 0) y[(b * T + t) * D + d] = r;
  }
  if (hf && dok) *reinterpret_cast<f32x4*>(hf + sidx) = h;
}

// Lanes that fill the GPU: 256 CUs x 8 waves x 64 lanes.
constexpr int64_t kFillThreads = 256LL * 8 * 64;

// The schedule a launch runs: the automatic choice streams when the lanes
// fill the GPU and goes chunk-parallel otherwise.  The workspace queries use
// the same functions, so a caller sizes exactly what the launch will read.
bool affd_chunked(int64_t S, int64_t nc, int32_t schedule) {
  if (schedule == CATOPT_SCAN_CHUNKED) return true;
  return schedule == CATOPT_SCAN_AUTO && nc > 1 && S < kFillThreads;
}

int64_t ssm_threads(int64_t B, int64_t D, int64_t N) {
  const int64_t tpd = N / 4;  // threads per channel (4 states per thread)
  const int64_t dpw = kThreads / tpd;
  return (D + dpw - 1) / dpw * kThreads * B;
}

bool ssm_chunked(int64_t B, int64_t D, int64_t N, int64_t nc, int32_t schedule) {
  if (schedule == CATOPT_SCAN_CHUNKED) return true;
  return schedule == CATOPT_SCAN_AUTO && nc > 1 && ssm_threads(B, D, N) < kFillThreads;
}

template <int N, bool APS>
int32_t ssm_launch(int64_t B, int64_t T, int64_t D, const float* a, const float* bx,
                   const float* c, const float* x, const float* h0, const int64_t* cs,
                   int64_t nc, int32_t schedule, float* y, float* hf, void* ws, int64_t wsb,
                   hipStream_t s) {
  const int64_t gx = (D + SsmLayout<N>::DPW - 1) / SsmLayout<N>::DPW;
  const int64_t S = B * D * N;
  static_assert(SsmLayout<N>::TPD == N / 4, "ssm_threads assumes four states per thread");
  const bool chunked = ssm_chunked(B, D, N, nc, schedule);
  if (gx > 0x7fffffff || B > 65535 || nc > 65535) return CATOPT_E_UNSUPPORTED;
  if constexpr (N == 16) {
    if (!chunked && APS) {
      ssm_stream_reg<N><<<dim3((uint32_t)gx, (uint32_t)B), dim3(kThreads), 0, s>>>(a, bx, c, x, h0, T, D, y, hf);
      CATOPT_LAUNCH_CHECK();
      return CATOPT_OK;
    }
  }
  if (!chunked && APS) {
    static bool attr_done = false;
    if (!attr_done) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&ssm_stream_lds<N>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, SsmLds<N>::BYTES);
      if (e != hipSuccess) return set_hip_error(e);
      attr_done = true;
    }
    ssm_stream_lds<N><<<dim3((uint32_t)gx, (uint32_t)B), dim3(kThreads), SsmLds<N>::BYTES, s>>>(
        a, bx, c, x, h0, T, D, y, hf);
    CATOPT_LAUNCH_CHECK();
    return CATOPT_OK;
  }
  if (!chunked) {
    ssm_stream<N, APS><<<dim3((uint32_t)gx, (uint32_t)B), dim3(kThreads), 0, s>>>(
        a, bx, c, x, h0, cs, nc, T, D, y, hf);
    CATOPT_LAUNCH_CHECK();
    return CATOPT_OK;
  }
  if (!ws || wsb < catopt_hip_scan_workspace_bytes(S, nc)) return CATOPT_E_WORKSPACE;
  float* ws_p = static_cast<float*>(ws);
  float* ws_h = ws_p + nc * S;
  ssm_chunk_local<N, APS><<<dim3((uint32_t)gx, (uint32_t)B, (uint32_t)nc), dim3(kThreads), 0, s>>>(
      a, bx, c, x, cs, T, D, S, ws_p, ws_h);
  CATOPT_LAUNCH_CHECK();
  scan_carry<<<dim3((uint32_t)((S + kThreads - 1) / kThreads)), dim3(kThreads), 0, s>>>(
      h0, nc, S, ws_p, ws_h, hf);
  CATOPT_LAUNCH_CHECK();
  ssm_chunk_apply<N, APS><<<dim3((uint32_t)gx, (uint32_t)B, (uint32_t)nc), dim3(kThreads), 0, s>>>(
      a, bx, c, x, cs, T, D, S, ws_h, y);
  CATOPT_LAUNCH_CHECK();
  return CATOPT_OK;
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int64_t catopt_hip_scan_workspace_bytes(int64_t S, int64_t n_chunks) {
  if (S < 0 || n_chunks < 0) return -1;
  return 2 * S * n_chunks * (int64_t)sizeof(float);
}

extern "C" int64_t catopt_hip_affd_scan_workspace_bytes(int64_t T, int64_t S, int64_t n_chunks,
                                                         int32_t schedule) {
  if (T < 0 || S < 0 || n_chunks < 1) return -1;
  if (schedule < CATOPT_SCAN_AUTO || schedule > CATOPT_SCAN_CHUNKED) return -1;
  return affd_chunked(S, n_chunks, schedule) ? catopt_hip_scan_workspace_bytes(S, n_chunks) : 0;
}

extern "C" int64_t catopt_hip_ssm_scan_workspace_bytes(int64_t B, int64_t T, int64_t D, int64_t N,
                                                        int64_t n_chunks, int32_t schedule) {
  if (B < 0 || T < 0 || D < 0 || n_chunks < 1) return -1;
  if (schedule < CATOPT_SCAN_AUTO || schedule > CATOPT_SCAN_CHUNKED) return -1;
  if (N != 4 && N != 8 && N != 16 && N != 32 && N != 64) return -1;
  return ssm_chunked(B, D, N, n_chunks, schedule) ? catopt_hip_scan_workspace_bytes(B * D * N, n_chunks)
                                                  : 0;
}

namespace catopt {
namespace {

// Argument checks and launches of catopt_hip_affd_scan, with the workspace
// resolved by the caller: `ws_cap` is the bytes available at `ws` (a caller
// buffer, or the static scratch array of the no-allocation entry point).
int32_t affd_scan_body(int64_t T, int64_t S, const float* a, int64_t lda, const float* u,
                       int64_t ldu, const float* h0, const int64_t* chunk_starts,
                       int64_t n_chunks, int32_t schedule, float* states, float* h_final,
                       void* ws, int64_t ws_cap, hipStream_t s) {
  if (S > 0x7fffffffLL * kThreads || n_chunks > 65535) return CATOPT_E_UNSUPPORTED;
  const int64_t gx = (S + kThreads - 1) / kThreads;
  const bool chunked = affd_chunked(S, n_chunks, schedule);
  if (!chunked) {
    affd_stream<<<dim3((uint32_t)gx), dim3(kThreads), 0, s>>>(a, lda, u, ldu, h0, chunk_starts,
                                                              n_chunks, T, S, states, h_final);
    CATOPT_LAUNCH_CHECK();
    return CATOPT_OK;
  }
  if (!ws || ws_cap < catopt_hip_scan_workspace_bytes(S, n_chunks)) return CATOPT_E_WORKSPACE;
  float* ws_p = static_cast<float*>(ws);
  float* ws_h = ws_p + n_chunks * S;
  affd_chunk_local<<<dim3((uint32_t)gx, (uint32_t)n_chunks), dim3(kThreads), 0, s>>>(
      a, lda, u, ldu, chunk_starts, T, S, ws_p, ws_h);
  CATOPT_LAUNCH_CHECK();
  scan_carry<<<dim3((uint32_t)gx), dim3(kThreads), 0, s>>>(h0, n_chunks, S, ws_p, ws_h, h_final);
  CATOPT_LAUNCH_CHECK();
  if (states) {
    affd_chunk_apply<<<dim3((uint32_t)gx, (uint32_t)n_chunks), dim3(kThreads), 0, s>>>(
        a, lda, u, ldu, chunk_starts, T, S, ws_h, states);
    CATOPT_LAUNCH_CHECK();
  }
  return CATOPT_OK;
}

int32_t affd_scan_args_ok(int64_t T, int64_t S, const float* a, int64_t lda, const float* u,
                          int64_t ldu, const int64_t* chunk_starts, int64_t n_chunks,
                          int32_t schedule) {
  if (T < 0 || S < 0 || n_chunks < 1 || lda < 0 || ldu < S) return CATOPT_E_INVAL;
  if (lda != 0 && lda < S) return CATOPT_E_INVAL;
  if (schedule < CATOPT_SCAN_AUTO || schedule > CATOPT_SCAN_CHUNKED) return CATOPT_E_INVAL;
  if (S > 0 && (!chunk_starts || (T > 0 && (!a || !u)))) return CATOPT_E_INVAL;
  return CATOPT_OK;
}

// Scratch of the no-allocation entry point: a file-scope device array that
// each GPU holds from the library's load to the end of the process.  Its
// name is a host-side stand-in, not a device address: host code uses only
// the per-device address that hipGetSymbolAddress returns for it.  The
// chunk-parallel schedule writes every word it later reads (chunk maps and
// local states, then the carries), so nothing in it has to start at zero.
constexpr int64_t kAffdScratchBytes = CATOPT_AFFD_SCAN_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kAffdScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The address of `scratch` on the stream's device, looked up once per
// device with that device current (made current for the lookup when the
// caller's current device is another one, then restored).
int32_t affd_scratch(hipStream_t stream, void** out) {
  hipDevice_t dev = -1;
  hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) return set_hip_error(e);
  if (dev < 0 || dev >= kMaxDevices) return CATOPT_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return set_hip_error(e);
    if (cur != dev) {
      e = hipSetDevice(dev);
      if (e != hipSuccess) return set_hip_error(e);
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return set_hip_error(e);
    if (back != hipSuccess) return set_hip_error(back);
    if (!p) return CATOPT_E_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CATOPT_OK;
}

}  // namespace
}  // namespace catopt

extern "C" int32_t catopt_hip_affd_scan(int64_t T, int64_t S, const float* a, int64_t lda,
                                        const float* u, int64_t ldu, const float* h0,
                                        const int64_t* chunk_starts, int64_t n_chunks,
                                        int32_t schedule, float* states, float* h_final,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  const int32_t st = affd_scan_args_ok(T, S, a, lda, u, ldu, chunk_starts, n_chunks, schedule);
  if (st != CATOPT_OK) return st;
  if (S == 0) return CATOPT_OK;
  return affd_scan_body(T, S, a, lda, u, ldu, h0, chunk_starts, n_chunks, schedule, states, h_final,
                        workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int64_t catopt_hip_affd_scan_noalloc_max_bytes(void) { return kAffdScratchBytes; }

extern "C" int32_t catopt_hip_affd_scan_noalloc(int64_t T, int64_t S, const float* a, int64_t lda,
                                                const float* u, int64_t ldu, const float* h0,
                                                const int64_t* chunk_starts, int64_t n_chunks,
                                                int32_t schedule, float* states, float* h_final,
                                                void* stream) {
  int32_t st = affd_scan_args_ok(T, S, a, lda, u, ldu, chunk_starts, n_chunks, schedule);
  if (st != CATOPT_OK) return st;
  if (S == 0) return CATOPT_OK;
  void* ws = nullptr;
  if (affd_chunked(S, n_chunks, schedule)) {
    // reject before touching the device: the chunked workspace must fit
    if (catopt_hip_scan_workspace_bytes(S, n_chunks) > kAffdScratchBytes) return CATOPT_E_WORKSPACE;
    st = affd_scratch(static_cast<hipStream_t>(stream), &ws);
    if (st != CATOPT_OK) return st;
  }
  return affd_scan_body(T, S, a, lda, u, ldu, h0, chunk_starts, n_chunks, schedule, states, h_final,
                        ws, ws ? kAffdScratchBytes : 0, static_cast<hipStream_t>(stream));
}

extern "C" int32_t catopt_hip_ssm_scan(int64_t B, int64_t T, int64_t D, int64_t N,
                                       const float* a, int32_t a_per_state, const float* bx,
                                       const float* c, const float* x, const float* h0,
                                       const int64_t* chunk_starts, int64_t n_chunks,
                                       int32_t schedule, float* y, float* h_final,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  if (B < 0 || T < 0 || D < 0 || n_chunks < 1) return CATOPT_E_INVAL;
  if (schedule < CATOPT_SCAN_AUTO || schedule > CATOPT_SCAN_CHUNKED) return CATOPT_E_INVAL;
  if (B == 0 || D == 0) return CATOPT_OK;
  if (!chunk_starts || (T > 0 && (!a || !bx || !c || !x || !y))) return CATOPT_E_INVAL;
  if (!aligned16(a) && a_per_state) return CATOPT_E_INVAL;
  if (!aligned16(bx) || !aligned16(c) || (h0 && !aligned16(h0)) || (h_final && !aligned16(h_final)))
    return CATOPT_E_INVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define CATOPT_SSM(NN)                                                                                \
  case NN:                                                                                            \
    return a_per_state ? ssm_launch<NN, true>(B, T, D, a, bx, c, x, h0, chunk_starts, n_chunks,     \
                                              schedule, y, h_final, workspace, workspace_bytes, s)  \
                       : ssm_launch<NN, false>(B, T, D, a, bx, c, x, h0, chunk_starts, n_chunks,    \
                                               schedule, y, h_final, workspace, workspace_bytes, s);
  switch (N) {
    CATOPT_SSM(4)
    CATOPT_SSM(8)
    CATOPT_SSM(16)
    CATOPT_SSM(32)
    CATOPT_SSM(64)
    default:
      return CATOPT_E_UNSUPPORTED;
  }
#undef CATOPT_SSM
}
