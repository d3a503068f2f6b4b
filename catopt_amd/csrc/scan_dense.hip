// Dense affine scans on gfx950 (fp32, MFMA).
//
//   X_t = A_t X_{t-1} + b_t 1ᵀ        t = 0 … T-1,  X_{-1} = h0
//
// Each of P slots carries a d x k state (d ≤ 64); A_t is d x d, b_t a
// d-vector added to every column.  Columns never mix under the update, so
// the scan is batched over columns: one wave owns 16 columns of one map
// group and keeps them as d/16 MFMA accumulator tiles (v_mfma_f32_16x16x4_f32,
// lane l holds rows 16·tile + 4·(l/16) + i, i = 0..3, of column l%16).
//
// One step is (d/16)² x 4 MFMAs whose B operands are the previous step's
// accumulators as they sit: register i of tile kb is, lane for lane, the B
// operand of a 16x16x4 product over the k indices {16·kb + 4j + i : j=0..3}
// (lane l supplies B[k = l/16][n = l%16]).  The matching A operand is
// A_t[16·rb + l%16][16·kb + 4·(l/16) + i]: for i = 0..3 four consecutive
// floats, one 16-byte load per tile pair.  No LDS, no lane shuffles; b_t
// enters as the accumulator's initial value.
//
// Map groups: when every slot shares one map sequence (lda_p = 0) all P·k
// columns form one group, and a step is one GEMM with N = P·k (the LTI
// system and a shared time-varying one); otherwise each slot is its own
// group of k columns and the kernel streams that slot's A_t from HBM.
//
// Schedules (chunk table as for the diagonal scans):
//   STREAM  — every wave walks all T steps; inputs are read once.
//   CHUNKED — (1) every chunk composes its own map (M_c, v_c) from the
//             identity: the same step run over the columns [I | 0] with b
//             added only to the v columns (one per slot); (2) the carries
//             fold over the chunks in table order: the same step again with
//             A = M_c, b = v_c, leaving the state after each chunk in the
//             workspace; (3) every chunk re-runs from its carry-in and
//             writes its prefix states (only when states are requested).
//             The two-level blocked scan of the reference's all-prefix path,
//             for systems whose columns alone cannot fill the GPU.
#include "common.hpp"

namespace catopt {
namespace {

constexpr int kWaves = 4;  // independent waves per workgroup (no LDS, no barriers)

struct DenseScan {
  const float* A;
  int64_t lda_t, lda_p;  // map of (step t, group g) at A + t·lda_t + g·lda_p (row-major d x d)
  const float* b;
  int64_t ldb_t, ldb_p;  // b of (step t, slot p) at b + t·ldb_t + p·ldb_p
  const float* h0;       // (P, d, k) or null (zeros)
  const float* carry;    // chunked re-scan: state entering chunk c ≥ 1 at carry + (c-1)·P·d·k
  float* states;         // (steps, P, d, k): row t = state after step t
  float* hf;             // (P, d, k)
  float* ws_m;           // chunk maps (n_chunks, G, d, d)
  float* ws_v;           // chunk offsets (n_chunks, P, d)
  int64_t P, d, k;
  int shared;            // one map group for all slots
};

__device__ __forceinline__ int64_t cclamp_d(int64_t v, int64_t T) { return v < 0 ? 0 : (v > T ? T : v); }

// Where a lane's column lives.  MAP mode columns are [identity d | v]; the v
// columns are one per slot (shared group) or the slot's own (per-slot group).
struct Col {
  int64_t p;  // slot (for b, h0, states); valid only if live
  int64_t j;  // state column within the slot (STATE) / map column (MAP, < d)
  bool live;  // inside the group's columns
  bool aff;   // receives b
  bool map;   // identity column of a chunk map (MAP mode)
};

template <bool MAP>
__device__ __forceinline__ Col column_of(const DenseScan& s, int64_t g, int64_t c) {
  Col r{0, 0, false, false, false};
  if (!MAP) {
    const int64_t ncols = s.shared ? s.P * s.k : s.k;
    if (c >= ncols) return r;
    r.live = r.aff = true;
    r.p = s.shared ? c / s.k : g;
    r.j = s.shared ? c % s.k : c;
    return r;
  }
  const int64_t nv = s.shared ? s.P : 1;
  if (c >= s.d + nv) return r;
  r.live = true;
  if (c < s.d) {
    r.map = true;
    r.j = c;
  } else {
    r.aff = true;
    r.p = s.shared ? c - s.d : g;
  }
  return r;
}

template <int DT, bool AT>
struct Frag {
  f32x4 a[AT ? DT * DT : 1];
  f32x4 b[DT];
};

// FULL: d = 16·DT and every A / b row starts 16-byte aligned (vector loads).
template <int DT, bool FULL>
__device__ __forceinline__ void load_a(f32x4* af, const float* __restrict__ At, int64_t d, int lane) {
#pragma unroll
  for (int rb = 0; rb < DT; ++rb) {
#pragma unroll
    for (int kb = 0; kb < DT; ++kb) {
      const int64_t row = rb * 16 + (lane & 15), col = kb * 16 + 4 * (lane >> 4);
      if (FULL) {
        af[rb * DT + kb] = *reinterpret_cast<const f32x4*>(At + row * d + col);
      } else {
        f32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (row < d && col + i < d) ? At[row * d + col + i] : 0.f;
        af[rb * DT + kb] = v;
      }
    }
  }
}

// Every lane loads (columns without b read slot 0's offsets, which exist);
// the rows past d and the columns without b are zeroed where the values are
// used (dense_step), not here: a select right after the load would make the
// wave wait for the prefetch it has just issued.
template <int DT, bool FULL>
__device__ __forceinline__ void load_b(f32x4* bf, const float* __restrict__ bt, int64_t d, int lane) {
#pragma unroll
  for (int rb = 0; rb < DT; ++rb) {
    const int64_t row0 = rb * 16 + 4 * (lane >> 4);
    f32x4 v;
    if (FULL) {
      v = *reinterpret_cast<const f32x4*>(bt + row0);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = bt[row0 + i < d ? row0 + i : d - 1];
    }
    bf[rb] = v;
  }
}

template <int DT, bool AT, bool FULL>
__device__ __forceinline__ void load_step(Frag<DT, AT>& f, const DenseScan& s, int64_t t, int64_t g,
                                          const Col& col, int lane) {
  if (AT) load_a<DT, FULL>(f.a, s.A + t * s.lda_t + g * s.lda_p, s.d, lane);
  load_b<DT, FULL>(f.b, s.b + t * s.ldb_t + (col.aff ? col.p : 0) * s.ldb_p, s.d, lane);
}

// X ← A·X + b over one step (accumulator tiles x[kb], see the file header).
// MASKED: b enters only columns with aff set and rows below d (chunk-map
// identity columns, padded tiles); otherwise every column takes b as loaded
// (columns past the group's end are never stored).
template <int DT, bool MASKED>
__device__ __forceinline__ void dense_step(f32x4* x, const f32x4* af, const f32x4* bf, bool aff, int64_t d,
                                           int lane) {
  f32x4 nx[DT];
#pragma unroll
  for (int rb = 0; rb < DT; ++rb) {
    if (MASKED) {
#pragma unroll
      for (int i = 0; i < 4; ++i) nx[rb][i] = (aff && rb * 16 + 4 * (lane >> 4) + i < d) ? bf[rb][i] : 0.f;
    } else {
      nx[rb] = bf[rb];
    }
  }
#pragma unroll
  for (int kb = 0; kb < DT; ++kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int rb = 0; rb < DT; ++rb)
        nx[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[rb * DT + kb][i], x[kb][i], nx[rb], 0, 0, 0);
    }
  }
#pragma unroll
  for (int rb = 0; rb < DT; ++rb) x[rb] = nx[rb];
}

// Stores the lane's rows of a (P, d, k) state image at base (STATE mode).
template <int DT, bool FULL>
__device__ __forceinline__ void store_state(float* __restrict__ base, const f32x4* x, const DenseScan& s,
                                            const Col& col, int lane) {
  if (!col.live) return;
#pragma unroll
  for (int rb = 0; rb < DT; ++rb) {
    const int64_t row0 = rb * 16 + 4 * (lane >> 4);
    if (FULL && s.k == 1) {
      *reinterpret_cast<f32x4*>(base + col.p * s.d + row0) = x[rb];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (row0 + i < s.d) base[(col.p * s.d + row0 + i) * s.k + col.j] = x[rb][i];
    }
  }
}

// Steps a block holds in flight per wave: enough loads to cover HBM latency
// at every tile count, within the register budget.
template <int DT, bool AT>
struct Unroll {
  static constexpr int U = AT ? (DT == 1 ? 8 : DT == 2 ? 2 : 1) : (DT == 1 ? 8 : DT == 2 ? 4 : 2);
};

// What a launch computes (phases of the header's schedules):
//   STREAM_FINAL — [0, T) from h0, the last state only;
//   STREAM_ALL   — [0, T) from h0, every state and the last;
//   MAP          — chunk blockIdx.y's map (M_c, v_c) from the identity;
//   RESCAN       — chunk blockIdx.y from its carry-in, every state.
// (plain ints, so kernel names stay readable in profiles: aff_dense_scan<DT, AT, FULL, MODE>)
namespace Mode {
constexpr int STREAM_FINAL = 0, STREAM_ALL = 1, MAP = 2, RESCAN = 3;
}

// Steps [t0, t1) in blocks of U: two fragment sets alternate, so the loads
// of block n+1 are issued before block n's products and consumed in place
// (a copy from a prefetch buffer would make the compiler wait for the
// prefetch at the copy).  The prefetch never branches: past the last block
// it re-reads a block in range.
template <int DT, bool AT, bool FULL, bool EMIT, bool MASKED>
__device__ __forceinline__ void run_steps(f32x4* x, const f32x4* a_lti, const DenseScan& s, int64_t g,
                                          const Col& col, int lane, int64_t t0, int64_t t1) {
  constexpr int U = Unroll<DT, AT>::U;
  const int64_t slot_stride = s.P * s.d * s.k;
  Frag<DT, AT> fa[U], fb[U];
  auto load_blk = [&](Frag<DT, AT>* f, int64_t tb) {
#pragma unroll
    for (int u = 0; u < U; ++u) load_step<DT, AT, FULL>(f[u], s, tb + u, g, col, lane);
  };
  auto run_blk = [&](const Frag<DT, AT>* f, int64_t tb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      dense_step<DT, MASKED>(x, AT ? f[u].a : a_lti, f[u].b, col.aff, s.d, lane);
      if (EMIT) store_state<DT, FULL>(s.states + (tb + u) * slot_stride, x, s, col, lane);
    }
  };
  const int64_t nblk = (t1 - t0) / U;
  int64_t t = t0, blk = 0;
  if (nblk > 0) load_blk(fa, t);
  for (; blk + 2 <= nblk; blk += 2, t += 2 * U) {
    load_blk(fb, t + U);
    __builtin_amdgcn_sched_barrier(0);
    run_blk(fa, t);
    __builtin_amdgcn_sched_barrier(0);
    load_blk(fa, blk + 2 < nblk ? t + 2 * U : t + U);
    __builtin_amdgcn_sched_barrier(0);
    run_blk(fb, t + U);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (blk < nblk) {
    run_blk(fa, t);
    t += U;
  }
  for (; t < t1; ++t) {
    Frag<DT, AT> f;
    load_step<DT, AT, FULL>(f, s, t, g, col, lane);
    dense_step<DT, MASKED>(x, AT ? f.a : a_lti, f.b, col.aff, s.d, lane);
    if (EMIT) store_state<DT, FULL>(s.states + t * slot_stride, x, s, col, lane);
  }
}

// grid: x = ⌈jobs / kWaves⌉ (job = group x 16-column tile), y = chunk (or 1).
template <int DT, bool AT, bool FULL, int M>
__global__ __launch_bounds__(64 * kWaves) void aff_dense_scan(DenseScan s, const int64_t* __restrict__ cs,
                                                              int64_t T, int64_t tiles, int64_t jobs) {
  constexpr bool MAP = M == Mode::MAP;
  constexpr bool CHUNKED = M == Mode::MAP || M == Mode::RESCAN;
  constexpr bool EMIT = M == Mode::STREAM_ALL || M == Mode::RESCAN;
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (job >= jobs) return;  // whole wave
  const int64_t g = job / tiles, c = (job % tiles) * 16 + (lane & 15);
  const Col col = column_of<MAP>(s, g, c);
  const int64_t chunk = CHUNKED ? (int64_t)blockIdx.y : 0;
  const int64_t t0 = CHUNKED ? cclamp_d(cs[chunk], T) : 0;
  const int64_t t1 = CHUNKED ? cclamp_d(cs[chunk + 1], T) : T;

  // initial state
  f32x4 x[DT];
  const float* init = s.h0;
  if (M == Mode::RESCAN && chunk > 0) init = s.carry + (chunk - 1) * s.P * s.d * s.k;
#pragma unroll
  for (int rb = 0; rb < DT; ++rb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = rb * 16 + 4 * (lane >> 4) + i;
      float v = 0.f;
      if (MAP) {
        v = (col.map && row == col.j) ? 1.f : 0.f;
      } else if (col.live && init && row < s.d) {
        v = init[(col.p * s.d + row) * s.k + col.j];
      }
      x[rb][i] = v;
    }
  }

  f32x4 a_lti[AT ? 1 : DT * DT];
  if (!AT) load_a<DT, FULL>(a_lti, s.A + g * s.lda_p, s.d, lane);
  run_steps<DT, AT, FULL, EMIT, MAP || !FULL>(x, a_lti, s, g, col, lane, t0, t1);

  if (MAP) {
    if (!col.live) return;
    const int64_t G = s.shared ? 1 : s.P;
#pragma unroll
    for (int rb = 0; rb < DT; ++rb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = rb * 16 + 4 * (lane >> 4) + i;
        if (row >= s.d) continue;
        if (col.map)
          s.ws_m[((chunk * G + g) * s.d + row) * s.d + col.j] = x[rb][i];
        else
          s.ws_v[(chunk * s.P + col.p) * s.d + row] = x[rb][i];
      }
    }
    return;
  }
  if (s.hf) store_state<DT, FULL>(s.hf, x, s, col, lane);
}

// Waves that fill the GPU once: 256 CUs x one wave per CU.
constexpr int64_t kFillWaves = 256;

struct WsLayout {
  int64_t m, v, carry, total;  // float offsets (256-byte aligned) and total floats
};

WsLayout ws_layout(int64_t P, int64_t d, int64_t k, bool shared, int64_t nc) {
  auto up = [](int64_t n) { return (n + 63) / 64 * 64; };
  WsLayout w;
  w.m = 0;
  w.v = up(nc * (shared ? 1 : P) * d * d);
  w.carry = w.v + up(nc * P * d);
  w.total = w.carry + up(nc * P * d * k);
  return w;
}

template <int DT, bool AT, bool FULL, int M>
void launch_one(const DenseScan& s, const int64_t* cs, int64_t T, int64_t tiles, int64_t jobs, int64_t ny,
                hipStream_t st) {
  const dim3 grid((uint32_t)((jobs + kWaves - 1) / kWaves), (uint32_t)ny);
  aff_dense_scan<DT, AT, FULL, M><<<grid, dim3(64 * kWaves), 0, st>>>(s, cs, T, tiles, jobs);
}

template <int DT, bool AT, bool FULL>
int32_t dense_launch(DenseScan s, int64_t T, const int64_t* cs, int64_t nc, int32_t schedule, void* ws,
                     int64_t wsb, hipStream_t st) {
  const int64_t G = s.shared ? 1 : s.P;
  const int64_t tiles_state = s.shared ? (s.P * s.k + 15) / 16 : (s.k + 15) / 16;
  const int64_t jobs_state = G * tiles_state;
  bool chunked = schedule == CATOPT_SCAN_CHUNKED;
  if (schedule == CATOPT_SCAN_AUTO) chunked = nc > 1 && T >= 256 && jobs_state < kFillWaves;
  if (jobs_state > 0x7fffffffLL * kWaves) return CATOPT_E_UNSUPPORTED;
  if (!chunked) {
    if (s.states)
      launch_one<DT, AT, FULL, Mode::STREAM_ALL>(s, cs, T, tiles_state, jobs_state, 1, st);
    else
      launch_one<DT, AT, FULL, Mode::STREAM_FINAL>(s, cs, T, tiles_state, jobs_state, 1, st);
    CATOPT_LAUNCH_CHECK();
    return CATOPT_OK;
  }
  const WsLayout w = ws_layout(s.P, s.d, s.k, s.shared != 0, nc);
  if (!ws || wsb < w.total * (int64_t)sizeof(float)) return CATOPT_E_WORKSPACE;
  float* wf = static_cast<float*>(ws);
  // (1) chunk maps
  DenseScan m = s;
  m.ws_m = wf + w.m;
  m.ws_v = wf + w.v;
  m.states = nullptr;
  m.hf = nullptr;
  const int64_t tiles_map = s.shared ? (s.d + s.P + 15) / 16 : (s.d + 1 + 15) / 16;
  if (G * tiles_map > 0x7fffffffLL * kWaves) return CATOPT_E_UNSUPPORTED;
  launch_one<DT, AT, FULL, Mode::MAP>(m, cs, T, tiles_map, G * tiles_map, nc, st);
  CATOPT_LAUNCH_CHECK();
  // (2) carries: A = M_c, b = v_c over the n_chunks "steps"
  DenseScan c = s;
  c.A = m.ws_m;
  c.lda_t = G * s.d * s.d;
  c.lda_p = s.shared ? 0 : s.d * s.d;
  c.b = m.ws_v;
  c.ldb_t = s.P * s.d;
  c.ldb_p = s.d;
  c.states = s.states ? wf + w.carry : nullptr;
  // FULL implies d = 16·DT: the workspace rows are then 16-byte aligned too
  if (c.states)
    launch_one<DT, true, FULL, Mode::STREAM_ALL>(c, cs, nc, tiles_state, jobs_state, 1, st);
  else
    launch_one<DT, true, FULL, Mode::STREAM_FINAL>(c, cs, nc, tiles_state, jobs_state, 1, st);
  CATOPT_LAUNCH_CHECK();
  // (3) prefix states from each chunk's carry-in
  if (s.states) {
    DenseScan r = s;
    r.carry = wf + w.carry;
    r.hf = nullptr;
    launch_one<DT, AT, FULL, Mode::RESCAN>(r, cs, T, tiles_state, jobs_state, nc, st);
    CATOPT_LAUNCH_CHECK();
  }
  return CATOPT_OK;
}

template <int DT>
int32_t dense_dispatch(const DenseScan& s, bool at, bool full, int64_t T, const int64_t* cs, int64_t nc,
                       int32_t schedule, void* ws, int64_t wsb, hipStream_t st) {
  if (at)
    return full ? dense_launch<DT, true, true>(s, T, cs, nc, schedule, ws, wsb, st)
                : dense_launch<DT, true, false>(s, T, cs, nc, schedule, ws, wsb, st);
  return full ? dense_launch<DT, false, true>(s, T, cs, nc, schedule, ws, wsb, st)
              : dense_launch<DT, false, false>(s, T, cs, nc, schedule, ws, wsb, st);
}

}  // namespace
}  // namespace catopt

using namespace catopt;

extern "C" int64_t catopt_hip_aff_scan_workspace_bytes(int64_t P, int64_t d, int64_t k, int32_t shared_map,
                                                       int64_t n_chunks) {
  if (P < 0 || d < 0 || k < 0 || n_chunks < 0) return -1;
  return ws_layout(P, d, k, shared_map != 0, n_chunks).total * (int64_t)sizeof(float);
}

extern "C" int32_t catopt_hip_aff_scan(int64_t T, int64_t P, int64_t d, int64_t k, const float* A,
                                       int64_t lda_t, int64_t lda_p, const float* b, int64_t ldb_t,
                                       int64_t ldb_p, const float* h0, const int64_t* chunk_starts,
                                       int64_t n_chunks, int32_t schedule, float* states, float* h_final,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  if (T < 0 || P < 0 || k < 1 || d < 1 || n_chunks < 1) return CATOPT_E_INVAL;
  if (lda_t < 0 || lda_p < 0 || ldb_t < 0 || ldb_p < 0) return CATOPT_E_INVAL;
  if (schedule < CATOPT_SCAN_AUTO || schedule > CATOPT_SCAN_CHUNKED) return CATOPT_E_INVAL;
  if (d > 64) return CATOPT_E_UNSUPPORTED;
  if (P == 0) return CATOPT_OK;
  if (!chunk_starts || !A || (T > 0 && !b)) return CATOPT_E_INVAL;
  if (n_chunks > 65535 || P > (1LL << 40) / (d * k)) return CATOPT_E_UNSUPPORTED;
  const int DT = (int)((d + 15) / 16);
  const bool full = d == 16 * DT && aligned16(A) && aligned16(b) && lda_t % 4 == 0 && lda_p % 4 == 0 &&
                    ldb_t % 4 == 0 && ldb_p % 4 == 0 && (!states || aligned16(states)) &&
                    (!h_final || aligned16(h_final));
  DenseScan s{};
  s.A = A;
  s.lda_t = lda_t;
  s.lda_p = lda_p;
  s.b = b;
  s.ldb_t = ldb_t;
  s.ldb_p = ldb_p;
  s.h0 = h0;
  s.states = states;
  s.hf = h_final;
  s.P = P;
  s.d = d;
  s.k = k;
  s.shared = lda_p == 0 ? 1 : 0;
  const bool at = lda_t != 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (DT) {
    case 1:
      return dense_dispatch<1>(s, at, full, T, chunk_starts, n_chunks, schedule, workspace, workspace_bytes, st);
    case 2:
      return dense_dispatch<2>(s, at, full, T, chunk_starts, n_chunks, schedule, workspace, workspace_bytes, st);
    case 3:
      return dense_dispatch<3>(s, at, full, T, chunk_starts, n_chunks, schedule, workspace, workspace_bytes, st);
    default:
      return dense_dispatch<4>(s, at, full, T, chunk_starts, n_chunks, schedule, workspace, workspace_bytes, st);
  }
}
