/*
 * catopt_hip.h — C ABI of libcatopt_hip.so, the MI355X (gfx950) executor
 * for the forms catopt's search delivers.
 *
 * The reference has no FFI on this path: its delivered forms run as eager
 * torch ops reached through Python bindings.  Each entry point below
 * replaces one binding (or one carrier-executor hot loop) of the reference;
 * the comment on each names the reference code it stands in for, as
 * path:line under luisfuturist/catopt.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers unless stated otherwise; sizes and
 *     strides are int64 element counts (not bytes).
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *     All work is enqueued on it; no entry point synchronises.
 *   - The return value is a catopt_status; 0 is success.  Nothing throws
 *     across the ABI.  On CATOPT_E_HIP the hipError_t is kept per thread
 *     and returned by catopt_hip_last_hip_error().
 *   - No entry point allocates device memory.  Workspace comes from the
 *     caller, sized by the matching *_workspace_bytes query.
 *   - State kept across calls: each kernel's maximum dynamic LDS is set on
 *     its first launch and the device's CU count is read once; both sit in
 *     function-static caches (idempotent; a concurrent first call writes
 *     the same values).  catopt_hip_affd_scan_noalloc uses a file-scope
 *     device array that each GPU holds until the process ends (see its
 *     entry).  Entry points are otherwise reentrant, and calls that share
 *     no output buffer may overlap on different streams.
 */
#ifndef CATOPT_HIP_H
#define CATOPT_HIP_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CATOPT_HIP_ABI_VERSION 1

/* status codes */
enum catopt_status {
  CATOPT_OK = 0,
  CATOPT_E_INVAL = 1,       /* bad argument: null pointer, size, stride, alignment */
  CATOPT_E_UNSUPPORTED = 2, /* valid request outside what the kernels cover (dtype, head dim) */
  CATOPT_E_HIP = 3,         /* a HIP runtime call failed (launch, attribute set) */
  CATOPT_E_WORKSPACE = 4    /* caller workspace smaller than *_workspace_bytes */
};

/* element types */
enum catopt_dtype {
  CATOPT_F32 = 0,
  CATOPT_BF16 = 1
};

/* GEMM epilogues (catopt_hip_linear) */
enum catopt_epilogue {
  CATOPT_EPI_NONE = 0,       /* y = x·wᵀ */
  CATOPT_EPI_BIAS = 1,       /* y = x·wᵀ + bias */
  CATOPT_EPI_BIAS_ADD2 = 2,  /* y = (x·wᵀ + bias) + bias2   (both [N] vectors) */
  CATOPT_EPI_SILU_MUL = 3,   /* y[:,n] = silu(x·w[n]ᵀ) * (x·w[n+N]ᵀ), w has 2N rows */
  CATOPT_EPI_GLU = 4         /* y[:,n] = (x·w[n]ᵀ) * sigmoid(x·w[n+N]ᵀ), w has 2N rows */
};

/* attention mask modes (catopt_hip_attn_fwd) */
enum catopt_mask_mode {
  CATOPT_MASK_NONE = 0,
  CATOPT_MASK_CAUSAL = 1,    /* keep key j for query i iff j <= i + causal_off */
  CATOPT_MASK_BOOL = 2,      /* keep where mask[i, j] != 0 (uint8 keep-mask) */
  CATOPT_MASK_BIAS = 3       /* add the fp32 bias mask[i, j] to scale·q·kᵀ (-inf masks) */
};

/* ABI version of the loaded library; equals CATOPT_HIP_ABI_VERSION. */
int32_t catopt_hip_abi_version(void);

/* Static text for a status code. */
const char* catopt_hip_strerror(int32_t status);

/* The hipError_t behind the last CATOPT_E_HIP on this thread (0 if none). */
int32_t catopt_hip_last_hip_error(void);

/*
 * RMSNorm over the last axis.
 *   y[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * w      (w may be NULL)
 * Arithmetic in fp32; x, w, y share `dtype`.  Rows are `ldx` / `ldy`
 * elements apart; columns are contiguous.
 * Replaces the "rms_norm" binding, torch_bridge.py:1404-1411, which the
 * RMS_NORM_FOLD law's RHS (laws/tensor.py:712-741) lowers through.
 */
int32_t catopt_hip_rmsnorm(int32_t dtype, int64_t rows, int64_t cols,
                           const void* x, int64_t ldx, const void* w,
                           float eps, void* y, int64_t ldy, void* stream);

/*
 * Linear layer with a fused epilogue:  y[M, Nout] = epi(x[M, K] · w[*, K]ᵀ).
 * x rows are `ldx` apart, w rows `ldw` apart (torch nn.Linear layout,
 * out_features × in_features), y rows `ldy` apart; the K axis of x and w
 * and the N axis of y are contiguous.  `N` is the output width; for
 * CATOPT_EPI_SILU_MUL / CATOPT_EPI_GLU, w holds 2N rows (the concat of the
 * two projections, first half then second half).  bias / bias2 are [N]
 * vectors of `dtype` (NULL unless the epilogue reads them).  fp32
 * accumulation.  bf16 with K-contiguous, 16-byte aligned operands and
 * K % 8 == 0 runs the persistent 16x16x32 bf16 MFMA kernel (one workgroup
 * per CU); other bf16 and all fp32 calls run 32x32x2 fp32 MFMA kernels.
 * Replaces the "linear" binding (torch_bridge.py:1251-1253), the bias adds
 * of the ASSOC_LINEAR_BIAS RHS (laws/tensor.py:1374-1394), and the
 * chunk/silu/mul (or glu) bindings of the SWIGLU_FUSE / GLU_FOLD RHS
 * (laws/tensor.py:1485-1519, 585-601; torch_bridge.py:1159,1310-1314,1631).
 */
int32_t catopt_hip_linear(int32_t dtype, int64_t M, int64_t N, int64_t K,
                          const void* x, int64_t ldx, const void* w,
                          int64_t ldw, const void* bias, const void* bias2,
                          int32_t epilogue, void* y, int64_t ldy,
                          void* stream);

/*
 * Batched matrix product with optional transposes:
 *   C[b] = op(A[b]) · op(B[b]),  op(X) = X or Xᵀ,  C[b] is M × N.
 * A[b] is M×K (transA=0, row stride lda) or K×M (transA=1); B[b] is K×N
 * (transB=0, row stride ldb) or N×K (transB=1).  Batch strides in
 * elements; a zero stride broadcasts.  fp32 or bf16, fp32 accumulation.
 * Replaces the "matmul" binding (torch_bridge.py:1147) as used by the
 * construction-time weight fold IRModule._fold_weight_chains
 * (torch_bridge.py:2451-2476) and by batched executor GEMMs.
 */
int32_t catopt_hip_matmul(int32_t dtype, int64_t batch, int64_t M, int64_t N,
                          int64_t K, const void* A, int64_t lda,
                          int64_t strideA, int32_t transA, const void* B,
                          int64_t ldb, int64_t strideB, int32_t transB,
                          void* C, int64_t ldc, int64_t strideC,
                          void* stream);

/*
 * Online-softmax attention forward over (batch, heads):
 *   s = scale · q kᵀ, masked entries set to -inf,
 *   (m, l, a) = (rowmax s, Σ exp(s - m), exp(s - m) · v)
 *   o = a / l           when normalize == 1   (om_apply: unclamped, a
 *                                              fully masked row gives NaN)
 *   o = a / l           when normalize == 2   (sdpa: a fully masked row
 *                                              gives 0)
 *   o = a               when normalize == 0   (the raw om numerator)
 * q: [B, H, Tq, d], k: [B, H, Tk, d], v: [B, H, Tk, dv], o: [B, H, Tq, dv];
 * the last axis is contiguous, the other three axes take explicit strides
 * (element counts, order b, h, t).  mask is a [Tq, Tk] plane with row
 * stride mask_ld, shared over (b, h): a uint8 keep-mask in mode
 * CATOPT_MASK_BOOL, an fp32 additive bias (4-byte aligned) in mode
 * CATOPT_MASK_BIAS — sdpa's float attn_mask, the attnbias(m) score term of
 * the explicit-mask form (om.py:1036-1050, 1315-1335).  m_out
 * and l_out (fp32, [B, H, Tq] contiguous) are optional: the om carriers
 * for om_compose with other key blocks.  bf16 only; d = dv = 128 or 64.
 * Replaces, for the OM_LIFT delivered form (om.py:153-193):
 * _om_elem (torch_bridge.py:1974-1981), _batched_elem (om_lower.py:462-472),
 * the om_compose level loop over key blocks (torch_bridge.py:1984-2006,
 * om_fused.py:51-96), the "om_apply" binding (torch_bridge.py:1890) and
 * the causal cmask / masked_fill bindings (om.py:1023-1029,
 * torch_bridge.py:1864).
 */
int32_t catopt_hip_attn_fwd(int32_t dtype, int64_t B, int64_t H, int64_t Tq,
                            int64_t Tk, int64_t d, int64_t dv,
                            const void* q, const int64_t* q_strides,
                            const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides,
                            float scale, int32_t mask_mode,
                            int64_t causal_off, const void* mask,
                            int64_t mask_ld, int32_t normalize, void* o,
                            const int64_t* o_strides, float* m_out,
                            float* l_out, void* stream);

/*
 * Row statistics of an explicit score block for the om element
 * (_om_elem, torch_bridge.py:1974-1981; _batched_elem, om_lower.py:
 * 462-472): for each row r of s [rows, cols] (fp32 or bf16, row stride lds)
 *   m[r] = max_c s[r, c]            (NaN when the row holds a NaN, as amax)
 *   e[r, c] = exp(s[r, c] - m[r]),  l[r] = Σ_c e[r, c]
 * in fp32 (e with row stride lde); a = e @ v then follows on the GEMM.
 * sanitize != 0 zeroes l and e on rows whose m is not finite (the leaf
 * sanitising of BatchedOMModule, om_lower.py:792-798); sanitize == 0 keeps
 * the raw binding's NaN for a fully masked row.
 */
int32_t catopt_hip_om_rows(int32_t dtype, int64_t rows, int64_t cols,
                           const void* s, int64_t lds, int32_t sanitize,
                           float* m, float* l, float* e, int64_t lde,
                           void* stream);

/*
 * Combine two om carriers (m, l, a) elementwise — the FlashAttention merge
 * with the isfinite guards of _om_compose (torch_bridge.py:1984-2006):
 *   mx = max(m1, m2) (NaN-propagating, as torch.maximum);
 *   e_i = isfinite(m_i) ? exp(m_i - mx) : 0;
 *   l = l1 e1 + l2 e2;  a = a1 e1 + a2 e2.
 * m, l: [rows] fp32; a: [rows, dv] fp32.  Outputs may alias input 1.
 */
int32_t catopt_hip_om_compose(int64_t rows, int64_t dv, const float* m1,
                              const float* l1, const float* a1,
                              const float* m2, const float* l2,
                              const float* a2, float* m, float* l, float* a,
                              void* stream);

/*
 * Chunked decayed retention (RetNet), the K-way delivered form
 * om_decayed_kway_blocks (om.py:3040-3210) executed by ChunkedDecayModule
 * (decayed_lower.py:381-724):
 *   o[t] = scale · Σ_{s ≤ t} γ_h^{t-s} (q[t]·k[s]) v[s]
 * evaluated chunk-wise: intra-chunk (q_i k_iᵀ ⊙ decay(γ, C)) v_i on MFMA,
 * inter-chunk through the state S_{i+1} = γ^C S_i + Σ_c γ^{C-c} k_ic ⊗ v_ic
 * carried across chunks (the rank-1 decay_vec factors of the cross blocks,
 * om.py:1075-1089).  q, k, v, o: [B, H, T, d] contiguous, 16-byte aligned,
 * all of dtype: CATOPT_BF16 (MFMA in bf16, state and accumulation in fp32;
 * d a multiple of 8 up to 128) or CATOPT_F32 (operands, products and state
 * in fp32; d a multiple of 4 up to 128); gamma: [H] fp32; chunk ∈ {64}; any
 * T (rows past T of the last chunk read as zeros and are not stored).
 * Workspace (bf16 only; the fp32 kernel takes none and ignores it):
 * catopt_hip_retention_workspace_bytes(...) bytes, any contents — the
 * per-segment start-state pieces when T is split into segments over the
 * current device's CUs, 0 when one segment per head fills the device
 * (without a device, the bound for the most segments any device takes).
 * -1 for an unsupported d / chunk.
 */
int64_t catopt_hip_retention_workspace_bytes(int64_t B, int64_t H, int64_t T,
                                             int64_t d, int64_t chunk);
int32_t catopt_hip_retention_fwd(int32_t dtype, int64_t B, int64_t H,
                                 int64_t T, int64_t d, int64_t chunk,
                                 const void* q, const void* k, const void* v,
                                 const float* gamma, float scale, void* o,
                                 void* workspace, int64_t workspace_bytes,
                                 void* stream);

/*
 * decay / decay_vec generators (om.py:1060-1089), fp32 on device:
 *   decay:     out[h, i, j] = γ_h^(i-j) for i ≥ j else 0      ([H, t, t])
 *   decay_vec: out[h, k]    = γ_h^(sign·k + offset)           ([H, t])
 */
int32_t catopt_hip_decay(int64_t H, int64_t t, const float* gamma,
                         float* out, void* stream);
int32_t catopt_hip_decay_vec(int64_t H, int64_t t, int64_t offset,
                             int64_t sign, const float* gamma, float* out,
                             void* stream);

/*
 * Read-only HBM stream over nbytes (a multiple of 16) of a 16-byte aligned
 * buffer: every byte is read once and nothing is written (sink, 4 bytes,
 * is stored only for one sentinel value of the data's XOR).  A measurement
 * kernel with no counterpart in the reference: the achievable read rate
 * against which the read-dominated scans are placed.
 */
int32_t catopt_hip_hbm_read(const void* src, int64_t nbytes, uint32_t* sink,
                            void* stream);

/* scan schedules (catopt_hip_affd_scan, catopt_hip_ssm_scan) */
enum catopt_scan_schedule {
  CATOPT_SCAN_AUTO = 0,       /* streaming when the lanes fill the GPU, else chunk-parallel */
  CATOPT_SCAN_STREAM = 1,     /* one pass: each lane walks the chunks in order */
  CATOPT_SCAN_CHUNKED = 2     /* chunk-parallel: local chunk maps, carry over chunks, re-scan */
};

/*
 * Diagonal affine scan over T steps of a state of S lanes (fp32):
 *   h_t = a_t ⊙ h_{t-1} + u_t,   h_{-1} = h0 (NULL = 0)
 * a, u: [T, S] with row strides lda, ldu (lda = 0 broadcasts one a row:
 * the LTI case).  states (optional, [T, S] contiguous) receives every
 * prefix state; h_final (optional, [S]) the last one.  The T steps are cut
 * into the chunks of the int64 table chunk_starts[0..n_chunks]
 * (chunk_starts[0] = 0, strictly ascending, chunk_starts[n_chunks] = T):
 * the chunk-parallel schedule composes each chunk's map independently,
 * folds the carries across chunks in table order, then re-applies each
 * chunk from its carry — the two-level blocked scan of
 * BatchedOmdModule._prefix_scan (omd_lower.py:771-824).  Workspace:
 * catopt_hip_scan_workspace_bytes(S, n_chunks) bytes for the
 * chunk-parallel schedule (0 is enough for streaming).
 * Replaces the diagonal-affine monoid's serial composition: the
 * aff_diag / affd_compose / applyd bindings (torch_bridge.py:1895-1900),
 * fused_diag_levels (scan_fused.py:100-120) and BatchedScanModule's diag
 * level loop (scan_lower.py:652-674).
 */
int64_t catopt_hip_scan_workspace_bytes(int64_t S, int64_t n_chunks);
/*
 * The bytes a catopt_hip_affd_scan call with these sizes and this schedule
 * reads from its workspace: the chunk-parallel size when that schedule runs
 * (CATOPT_SCAN_AUTO resolved exactly as the launch resolves it), else 0.
 * -1 for a bad size or schedule.
 */
int64_t catopt_hip_affd_scan_workspace_bytes(int64_t T, int64_t S, int64_t n_chunks,
                                             int32_t schedule);
int32_t catopt_hip_affd_scan(int64_t T, int64_t S, const float* a,
                             int64_t lda, const float* u, int64_t ldu,
                             const float* h0, const int64_t* chunk_starts,
                             int64_t n_chunks, int32_t schedule,
                             float* states, float* h_final, void* workspace,
                             int64_t workspace_bytes, void* stream);

/*
 * catopt_hip_affd_scan without a workspace argument: the one entry point
 * that allocates nothing and takes no caller workspace.  It has no
 * counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, and
 * harnesses that forbid hipMalloc.
 * Arguments, results and schedules are those of catopt_hip_affd_scan (the
 * same kernels run).  The chunk-parallel schedule keeps its chunk maps and
 * carries in a static device array of CATOPT_AFFD_SCAN_SCRATCH_BYTES
 * (16 MiB) that every GPU the library runs on holds until the process
 * ends; a call whose chunk-parallel workspace,
 * catopt_hip_scan_workspace_bytes(S, n_chunks), exceeds it returns
 * CATOPT_E_WORKSPACE before any device work.  Streaming calls use no
 * scratch.  All calls on one GPU share that GPU's array and leave their
 * contents in it: two calls that overlap on one GPU (streams not ordered
 * with each other) race, and the result of both is undefined.
 * The device address of the array is looked up once per device, on the
 * first call with that device current.
 */
#define CATOPT_AFFD_SCAN_SCRATCH_BYTES (16LL * 1024 * 1024)
int64_t catopt_hip_affd_scan_noalloc_max_bytes(void);
int32_t catopt_hip_affd_scan_noalloc(int64_t T, int64_t S, const float* a,
                                     int64_t lda, const float* u, int64_t ldu,
                                     const float* h0,
                                     const int64_t* chunk_starts,
                                     int64_t n_chunks, int32_t schedule,
                                     float* states, float* h_final,
                                     void* stream);

/*
 * Diagonal selective-SSM scan with the input and readout contractions
 * fused (the all-prefix stacked form gather_applyd_stack, xcarrier.py:
 * 2252-2273, read out by y_t = Σ_n c_t[n] h_t[·, n]):
 *   h[b,t,d,n] = a[b,t,d,n] · h[b,t-1,d,n] + bx[b,t,n] · x[b,t,d]
 *   y[b,t,d]   = Σ_n c[b,t,n] · h[b,t,d,n]
 * fp32; a: [B,T,D,N] contiguous (a_per_state = 1) or [B,T,D] broadcast
 * over N (a_per_state = 0); bx, c: [B,T,N]; x, y: [B,T,D]; h0, h_final:
 * [B,D,N] (optional, NULL h0 = 0).  N ∈ {4, 8, 16, 32, 64}; any D.  The
 * n-reduction runs across lanes with DPP/ds_swizzle shuffles.  Chunk table
 * and schedule as for catopt_hip_affd_scan; workspace for the
 * chunk-parallel schedule: catopt_hip_scan_workspace_bytes(B*D*N, n_chunks).
 */
/*
 * The bytes a catopt_hip_ssm_scan call with these sizes and this schedule
 * reads from its workspace (0 when it streams); -1 for a bad size, N or
 * schedule.
 */
int64_t catopt_hip_ssm_scan_workspace_bytes(int64_t B, int64_t T, int64_t D, int64_t N,
                                            int64_t n_chunks, int32_t schedule);
int32_t catopt_hip_ssm_scan(int64_t B, int64_t T, int64_t D, int64_t N,
                            const float* a, int32_t a_per_state,
                            const float* bx, const float* c, const float* x,
                            const float* h0, const int64_t* chunk_starts,
                            int64_t n_chunks, int32_t schedule, float* y,
                            float* h_final, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * fp32 attention carrier: the om element of the score block s = scale·q kᵀ
 * over values v whose width dv is independent of the key width dk,
 *   m = rowmax(s),  l = Σ_k exp(s − m),  a = Σ_k exp(s − m) v_k
 * per query row (the (m, l, a) triple of _om_elem, torch_bridge.py:1974-1981;
 * the deferred-affine omd_elem, xcarrier.py:380-400, with v = [fa | fb]).
 * q: [batch, Tq, dk] with batch stride q_sb and row stride ldq; k: [batch,
 * Tk, dk] (k_sb, ldk); v: [batch, Tk, dv] (v_sb, ldv; a stride of 0 shares
 * one block); m_out, l_out: [batch, Tq] contiguous; num: [batch, Tq, dv]
 * (num_sb, ldn).  A row with no finite score gets the empty carrier
 * (m = −∞, l = 0, a = 0).  dk ≤ 128, dv ≤ 256 (else CATOPT_E_UNSUPPORTED).
 * Replaces the score-block leaf of BatchedOmdModule's level loop
 * (omd_lower.py:885-898): the scores and exponentials stay on chip.
 */
int32_t catopt_hip_attn_carrier_f32(int64_t batch, int64_t Tq, int64_t Tk,
                                    int64_t dk, int64_t dv, const float* q,
                                    int64_t q_sb, int64_t ldq, const float* k,
                                    int64_t k_sb, int64_t ldk, const float* v,
                                    int64_t v_sb, int64_t ldv, float scale,
                                    float* m_out, float* l_out, float* num,
                                    int64_t num_sb, int64_t ldn, void* stream);

/*
 * catopt_hip_attn_carrier_f32 with a mask on the score block, in the modes
 * of catopt_hip_attn_fwd: CATOPT_MASK_CAUSAL keeps key j for query i iff
 * j <= i + causal_off (key tiles wholly past a query block are not read);
 * CATOPT_MASK_BOOL keeps where the uint8 plane mask[i, j] != 0;
 * CATOPT_MASK_BIAS adds the fp32 plane mask[i, j] (4-byte aligned) to the
 * scaled score, s = scale·q kᵀ + bias, as torch forms it (−inf masks; a row
 * biased by −FLT_MAX throughout keeps finite scores and weighs its keys as
 * torch does).  The plane is [Tq, Tk] with row stride mask_ld >= Tk, shared
 * over the batch.  A row whose keys are all masked gets the empty carrier.
 * Replaces, for fp32 operands, a masked score leaf of BatchedOMModule: the
 * score block with its cmask / masked_fill or attnbias term (om.py:1023-1050,
 * evaluated by _stacked_scores, om_lower.py:672-719) and _batched_elem
 * (om_lower.py:462-472) over it.
 */
int32_t catopt_hip_attn_carrier_f32_masked(
    int64_t batch, int64_t Tq, int64_t Tk, int64_t dk, int64_t dv,
    const float* q, int64_t q_sb, int64_t ldq, const float* k, int64_t k_sb,
    int64_t ldk, const float* v, int64_t v_sb, int64_t ldv, float scale,
    int32_t mask_mode, int64_t causal_off, const void* mask, int64_t mask_ld,
    float* m_out, float* l_out, float* num, int64_t num_sb, int64_t ldn,
    void* stream);

/*
 * The om combine of L carriers of one query block followed by the diagonal
 * deferred-affine readout, in one pass (fp32):
 *   M = max_i m_i (NaN-propagating, as amax), w_i = isfinite(m_i) ?
 *   exp(m_i − M) : 0, then out[r, c] = (Σ w_i fa_i[r, c] · h[c] +
 *   Σ w_i fb_i[r, c]) / Σ w_i l_i[r]
 * with fa_i, fb_i the two halves of num_i = [fa | fb].  m, l: [L, rows]
 * contiguous; num: [L, rows, ≥ 2d] (leaf stride num_sb, row stride ldn);
 * h: [d]; out: [rows, d] contiguous.  A row with no finite score in any
 * carrier is NaN (0 / 0), as the unclamped omd_apply gives it.
 * Replaces the level reduction and readout of BatchedOmdModule
 * (omd_lower.py:900-945 into fused_omd_levels, om_fused.py:151-164) when
 * every leaf's carrier comes from one catopt_hip_attn_carrier_f32 launch.
 */
int32_t catopt_hip_omd_fold_apply(int64_t L, int64_t rows, int64_t d,
                                  const float* m, const float* l,
                                  const float* num, int64_t ldn,
                                  int64_t num_sb, const float* h, float* out,
                                  void* stream);

/*
 * Dense affine scan over T steps of P slots, each carrying a d x k state
 * (fp32, 1 ≤ d ≤ 64, k ≥ 1):
 *   X_t[p] = A_t[p] · X_{t-1}[p] + b_t[p] 1ᵀ,   X_{-1} = h0 (NULL = 0)
 * A_t[p] is the row-major d x d block at A + t·lda_t + p·lda_p (lda_t = 0:
 * one map for every step, the LTI case; lda_p = 0: one map for every slot,
 * which batches all P·k columns into one MFMA product per step); b_t[p] the
 * d-vector at b + t·ldb_t + p·ldb_p, added to every column.  h0, h_final:
 * [P, d, k] contiguous; states (optional, [T, P, d, k]) receives every
 * prefix state.  Chunk table and schedule as for catopt_hip_affd_scan (the
 * chunk-parallel schedule composes each chunk's dense map from the
 * identity); its workspace: catopt_hip_aff_scan_workspace_bytes(P, d, k,
 * lda_p == 0, n_chunks) bytes (0 is enough for streaming).
 * d > 64: CATOPT_E_UNSUPPORTED.
 * Replaces the dense affine monoid's batched composition: the aff /
 * aff_compose / apply bindings (torch_bridge.py:1873-1881), the
 * homogeneous-matrix levels of BatchedScanModule (scan_lower.py:716-741,
 * 640-698) and fused_dense_levels (scan_fused.py:123-143), and the stacked
 * all-prefix form gather_apply_stack (xcarrier.py:2276-2293).
 */
int64_t catopt_hip_aff_scan_workspace_bytes(int64_t P, int64_t d, int64_t k,
                                            int32_t shared_map,
                                            int64_t n_chunks);
int32_t catopt_hip_aff_scan(int64_t T, int64_t P, int64_t d, int64_t k,
                            const float* A, int64_t lda_t, int64_t lda_p,
                            const float* b, int64_t ldb_t, int64_t ldb_p,
                            const float* h0, const int64_t* chunk_starts,
                            int64_t n_chunks, int32_t schedule, float* states,
                            float* h_final, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * One level of a compose forest over slot arrays (fp32).  Slots hold
 * affine maps: diagonal (A, B: [n_slots, S]) or dense (A: [n_slots, P, d,
 * d] row-major, B: [n_slots, P, d]).  For j < L (f, g: device int64[L]):
 *   slot[out0 + j] = compose(slot[f[j]], slot[g[j]])
 *   diagonal: (fa * ga, fa * gb + fb), product and sum rounded separately
 *   dense:    (fa @ ga, fa @ gb + fb)
 * Every f[j], g[j] must lie in [0, out0): an index outside gives NaN in
 * that output slot.  Requires 1 ≤ out0 ≤ n_slots and out0 + L ≤ n_slots.
 * Replaces the level loop of the forest plan of BatchedOmdModule
 * (omd_lower.py:849-866, plan 520-558) over _compose_pair
 * (omd_lower.py:236-246): one launch per level instead of per-node
 * affd_compose / aff_compose bindings (torch_bridge.py:1873-1900).
 */
int32_t catopt_hip_affd_compose_slots(int64_t n_slots, int64_t S, float* A,
                                      float* B, const int64_t* f,
                                      const int64_t* g, int64_t L,
                                      int64_t out0, void* stream);
int32_t catopt_hip_aff_compose_slots(int64_t n_slots, int64_t P, int64_t d,
                                     float* A, float* B, const int64_t* f,
                                     const int64_t* g, int64_t L,
                                     int64_t out0, void* stream);

/*
 * Elementwise helpers behind the generic evaluator's bindings when no
 * fused form applies: silu (torch_bridge.py:1159), mul (the "mul"
 * binding) and the paired silu·mul of SWIGLU_FUSE.  n elements,
 * contiguous, fp32 or bf16 (math in fp32).
 */
int32_t catopt_hip_silu(int32_t dtype, int64_t n, const void* x, void* y,
                        void* stream);
int32_t catopt_hip_silu_mul(int32_t dtype, int64_t n, const void* g,
                            const void* u, void* y, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CATOPT_HIP_H */
