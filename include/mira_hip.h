/* mira_hip.h -- C-ABI of the MI355X (gfx950) Mira mixer scan library, libmira_hip.so.
 *
 * This library replaces the reference's operator plugin for the mixer scan: the Python launcher
 * kernel/cuda/mira_dspv2/mira.py (matrix_lattice_iir :1439-1563, MatrixLatticeIIR.forward
 * :1149-1293) and its driver-API cubin loader kernel/cuda/driver.py (module_for :328-344,
 * launch_dims :910-934). Every entry point takes plain device pointers, element strides and sizes,
 * and the HIP stream to launch on (a hipStream_t passed as void*; NULL is the default stream).
 * Every launch is asynchronous on that stream; nothing synchronises the host.
 *
 * Return codes mirror the reference plugin's error conventions:
 *   MIRA_OK       0  launched
 *   MIRA_DECLINE  1  shape / dtype / layout this library does not serve -- the reference returns
 *                    None (mira.py:1450-1500) and the mixer raises RuntimeError
 *                    (model/mira_mixer.py:158-166, 822-824); there is no silent fallback
 *   MIRA_ERR_ARG  2  malformed argument (the reference's ValueError, mira.py:1505-1517)
 *   MIRA_ERR_HIP  3  a HIP launch failed (the reference's RuntimeError, mira.py:513-519)
 * mira_last_error() returns the message of the last failure on the calling thread.
 *
 * Element types (dtype): MIRA_F32, MIRA_BF16, MIRA_F16. Arithmetic is float32 throughout; states
 * are always float32. arch_mode is the reference kernel's stage mode of each stage-map arch
 * (kernel/cuda/mira_dspv2/mira.py:305-309): 3 cauchy_x_mobius, 6 cauchy_x_hyperbolic,
 * 7 cauchy_x_identity, 8-10 gaussian_x_{mobius,hyperbolic,identity}, 11-13 expexp_x_*,
 * 14-16 expsoftplus_x_*, 17-19 hill_x_*.
 */
#ifndef MIRA_HIP_H
#define MIRA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MIRA_OK = 0, MIRA_DECLINE = 1, MIRA_ERR_ARG = 2, MIRA_ERR_HIP = 3 };
enum { MIRA_F32 = 0, MIRA_BF16 = 1, MIRA_F16 = 2 };

/* Message of the last non-zero return on this thread ("" if none). */
const char *mira_last_error(void);

/* Library version string and the offload target it was built for ("gfx950"). */
const char *mira_version(void);

/* Whether (K, d_m, dtype) has compiled kernels: 1 yes, 0 no. The reference's ORDERS /
 * ORDER_MEMORIES table (kernel/cuda/mira_dspv2/mira.py:86,185-190). */
int mira_lattice_supported(int K, int M, int dtype);

/* ---------------------------------------------------------------------------------------------
 * The reference operator: the K-stage matrix lattice scan (model/mira_mixer.py:246-387).
 * Replaces the p1 -> tree scan -> p3 launch sequence of MatrixLatticeIIR.forward
 * (kernel/cuda/mira_dspv2/mira.py:1229-1276) for inference (no retained graph).
 *
 *   x      [B,T,C]     row stride x_row   (elements between consecutive tokens; batch stride T*x_row)
 *   alpha  [B,T,C,K]   row stride alpha_row, [C,K] tail dense
 *   beta   [B,T,C,K]   row stride beta_row,  [C,K] tail dense
 *   rho    [B,T,C,K+1] row stride rho_row,   [C,K+1] tail dense
 *   gamma  [B,T,C]     row stride gamma_row
 *   memory_write [B,T,M] contiguous (already SiLU'd)
 *   memory_read  [B,T,K+1,M] row stride read_row, [K+1,M] tail dense
 *   valid  [B,T] uint8 (0 = masked: state kept, output 0), or NULL
 *   state_in  [B,K,C,M] float32 or NULL (zeros);  state_out [B,K,C,M] float32 or NULL
 *   out    [B,T,C] contiguous, same dtype as x
 * chunk: tokens per chunk (0 = mira_lattice_plan_chunk's choice). workspace: device memory of at
 * least mira_lattice_workspace_bytes(B,T,C,K,M,chunk) bytes (may be NULL when that is 0).
 * state_out may not alias state_in. */
int mira_lattice_plan_chunk(int B, int T, int C, int K, int M);
size_t mira_lattice_workspace_bytes(int B, int T, int C, int K, int M, int chunk);
int mira_lattice_forward(const void *x, int64_t x_row, const void *alpha, int64_t alpha_row,
                         const void *beta, int64_t beta_row, const void *rho, int64_t rho_row,
                         const void *gamma, int64_t gamma_row, const void *memory_write,
                         const void *memory_read, int64_t read_row, const uint8_t *valid,
                         const float *state_in, float *state_out, void *out, int B, int T, int C,
                         int K, int M, int dtype, int arch_mode, int chunk, void *workspace,
                         size_t workspace_bytes, void *stream);

/* Allocation-free variant of mira_lattice_forward. It has no counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP-graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Arguments and results are mira_lattice_forward's
 * without the workspace: the chunk summaries live in a static device array of
 * MIRA_LATTICE_STATIC_SCRATCH_BYTES per GPU, which the library holds until the process ends; the
 * call allocates nothing and clears nothing (every scratch word it reads it wrote first). A call
 * whose chunk plan needs more than that (mira_lattice_workspace_bytes) returns MIRA_ERR_ARG;
 * pass a longer chunk (chunk = T needs none) or use mira_lattice_forward. All calls on one GPU
 * share the array, so calls that overlap in time on one GPU (two streams, two threads) race:
 * the caller must order them. */
#define MIRA_LATTICE_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
int mira_lattice_forward_static(const void *x, int64_t x_row, const void *alpha,
                                int64_t alpha_row, const void *beta, int64_t beta_row,
                                const void *rho, int64_t rho_row, const void *gamma,
                                int64_t gamma_row, const void *memory_write,
                                const void *memory_read, int64_t read_row, const uint8_t *valid,
                                const float *state_in, float *state_out, void *out, int B, int T,
                                int C, int K, int M, int dtype, int arch_mode, int chunk,
                                void *stream);

/* The backward (training): gradients of sum(grad_out * y) for y = mira_lattice_forward(...) with
 * respect to x, alpha, beta, rho, gamma, memory_write and memory_read. Replaces the b1 -> reverse
 * tree -> b3 -> b4 launches of MatrixLatticeIIR.backward (kernel/cuda/mira_dspv2/mira.py:
 * 1295-1433, backward.cuh) and the fine checkpoints its forward keeps (mira.py:1165-1170).
 *
 * The forward must have run with chunk = mira_lattice_backward_chunk(K, M) (0 when (K, M) has no
 * backward: the reference's ORDER_MEMORIES, K in {1,8} with d_m in {8,16}, K in {2,4} with
 * d_m in {8,16,32,64}); its workspace, which then holds every chunk's transition and the state
 * entering it, is passed back as forward_workspace (may be NULL when T <= that chunk), together
 * with the same inputs, valid mask and state_in. grad_out [B,T,C] is contiguous in x's dtype.
 * Every gradient is written in x's dtype at its own row stride (so the caller may point them at
 * views of packed projection gradients); with raw_write non-NULL ([B,T,M] at raw_write_row),
 * grad_write receives the gradient of the raw write, d/dz of SiLU(z) applied. workspace: at least
 * mira_lattice_backward_workspace_bytes(B,T,C,K,M) bytes, 16-byte aligned. */
int mira_lattice_backward_chunk(int K, int M);
size_t mira_lattice_backward_workspace_bytes(int B, int T, int C, int K, int M);
int mira_lattice_backward(const void *x, int64_t x_row, const void *alpha, int64_t alpha_row,
                          const void *beta, int64_t beta_row, const void *rho, int64_t rho_row,
                          const void *gamma, int64_t gamma_row, const void *memory_write,
                          const void *memory_read, int64_t read_row, const uint8_t *valid,
                          const float *state_in, const void *grad_out, void *grad_x,
                          int64_t grad_x_row, void *grad_alpha, int64_t grad_alpha_row,
                          void *grad_beta, int64_t grad_beta_row, void *grad_rho,
                          int64_t grad_rho_row, void *grad_gamma, int64_t grad_gamma_row,
                          void *grad_write, int64_t grad_write_row, const void *raw_write,
                          int64_t raw_write_row, void *grad_read, int64_t grad_read_row, int B,
                          int T, int C, int K, int M, int dtype, int arch_mode,
                          const void *forward_workspace, size_t forward_workspace_bytes,
                          void *workspace, size_t workspace_bytes, void *stream);

/* The decode step, T = 1: replaces mira_matrix_step_k{K}_m{M}_{dt}
 * (kernel/cuda/mira_dspv2/mira_iir.cu:376-411, launched at mira.py:1254-1276 when tokens == 1).
 * Same arguments as mira_lattice_forward at T = 1; no workspace. state_in and state_out may be
 * the same buffer (updated in place). */
int mira_lattice_step(const void *x, int64_t x_row, const void *alpha, int64_t alpha_row,
                      const void *beta, int64_t beta_row, const void *rho, int64_t rho_row,
                      const void *gamma, int64_t gamma_row, const void *memory_write,
                      const void *memory_read, int64_t read_row, const uint8_t *valid,
                      const float *state_in, float *state_out, void *out, int B, int C, int K,
                      int M, int dtype, int arch_mode, void *stream);

/* ---------------------------------------------------------------------------------------------
 * The inference scan that forms its own coefficients from the d_r-wide control: replaces
 * mira_fused_scan_k2_m16_r{16,32,48,64}_s{mode}_bf16 (kernel/cuda/mira_dspv2/fused_scan.cuh:259-516)
 * as launched by matrix_lattice_iir_control (kernel/cuda/mira_dspv2/mira.py:1675-1741). Every
 * coefficient is bf16(sum_k control[b,t,k] weight[row,k] + bias[row]), the mixer's
 * coefficient_projection rounded once to bf16; only the order of the d_r-term sum differs from a
 * GEMM's. The rows of weight (row stride weight_row, weight_rows rows) are
 *   alpha of (c, k): alpha_first + c K + k;  beta: beta_first + c K + k;
 *   rho of (c, k):   rho_first + c (K+1) + k   (k = 0..K)
 * and bias [weight_rows] (or NULL). control [B,T,R] contiguous; the other arguments are
 * mira_lattice_forward's, bf16 only; memory_read is the caller's projection of the control.
 * state_in and state_out may be the same buffer. mira_lattice_control_serves says whether a call
 * is served: bf16; (K, d_m) in {(1,8), (1,16), (2,8), (2,16), (4,8)} (the reference serves (2,16)),
 * where it is faster than the projection GEMM plus mira_lattice_forward; R in {16,32,48,64}; and
 * one token chunk covers the call, mira_lattice_plan_chunk(B,T,C,K,M) >= T (the reference's fused
 * plan asks for one inference chunk, mira.py:1642-1672). A call it does not serve returns
 * MIRA_DECLINE and the caller projects the coefficients and calls mira_lattice_forward
 * (mira.py:1693-1704). */
int mira_lattice_control_serves(int B, int T, int C, int K, int M, int R, int dtype);
int mira_lattice_control_forward(const void *x, int64_t x_row, const void *control,
                                 const void *weight, int64_t weight_row, int64_t weight_rows,
                                 const void *bias, int64_t alpha_first, int64_t beta_first,
                                 int64_t rho_first, const void *gamma, int64_t gamma_row,
                                 const void *memory_write, const void *memory_read,
                                 int64_t read_row, const uint8_t *valid, const float *state_in,
                                 float *state_out, void *out, int B, int T, int C, int K, int M,
                                 int R, int dtype, int arch_mode, void *stream);

/* ---------------------------------------------------------------------------------------------
 * BASELINE-literal depthwise causal conv (width W) + diagonal decay scan. No reference
 * counterpart (the reference mixer has no convolution, model/prefix_cache.py:14); it is the K=1,
 * M=1 lattice after the reparameterisation r = sqrt(a^2+(1-a)^2), alpha = -atanh(a/r),
 * beta = sqrt(1/r-1), with the conv applied to x first.
 *   u_t = sum_j w[d,j] x_(t-W+1+j) + bias[d];   h_t = a_t h_(t-1) + (1 - a_t) u_t;   y_t = h_t
 *   x, a, y [B,T,D] contiguous (dtype); w [D,W] float32; bias [D] float32 or NULL;
 *   h0 [B,D] float32 or NULL; hT [B,D] float32 or NULL (may equal h0);
 *   ring_in / ring_out [B,D,W-1] (dtype) or NULL: slot s holds x of the stream token t' = s
 *   (mod W-1) among the last W-1; pos = tokens the stream absorbed before this call. ring_out may
 *   equal ring_in.
 * Prefill is one pass over HBM. Where the batch has a 64-channel column for at least half the
 * CUs (B * ceil(D/64) >= CUs/2, e.g. BASELINE cfg2) one workgroup scans each column over all T
 * and the workspace is not touched; narrower batches split the tokens into tiles joined by a
 * decoupled look-back, whose workspace (mira_diag_workspace_bytes) must be zero-filled once when
 * first allocated and then only reused by calls on one stream at a time. The look-back form
 * refuses HIP-graph capture (MIRA_ERR_ARG): its per-launch epoch would be frozen into the graph.
 * W must be 4; D a multiple of 4. */
size_t mira_diag_workspace_bytes(int B, int T, int D, int dtype);
int mira_diag_conv_scan(const void *x, const void *a, const float *w, const float *bias,
                        const float *h0, const void *ring_in, void *ring_out, int64_t pos,
                        void *y, float *hT, int B, int T, int D, int W, int dtype,
                        void *workspace, size_t workspace_bytes, void *stream);
/* One decode token per sequence: x, a, y [B,D]; h [B,D] float32 updated in place; ring [B,D,W-1]
 * updated in place (one slot, pos mod (W-1), is rewritten). */
int mira_diag_conv_step(const void *x, const void *a, const float *w, const float *bias,
                        float *h, void *ring, int64_t pos, void *y, int B, int D, int W,
                        int dtype, void *stream);
/* Reads (synchronously) the look-back watchdog word of a diag workspace: 0 when every wait of
 * every prefill on it ended normally. */
int mira_diag_workspace_error(void *workspace, size_t workspace_bytes, unsigned *value);

/* ---------------------------------------------------------------------------------------------
 * BASELINE-literal gated linear attention (GLA) matrix state: per (b, head)
 *   S_t = exp(g_t) S_(t-1) + k_t v_t^T,   o_t = S_t^T q_t
 * the K=1 lattice with batch B*H, C = d_v, M = d_k (beta = 0, alpha = -atanh(e^g),
 * x = v / sqrt(1 - e^(2g)), s = k, nu = (q, 0)); the state is stored as the lattice state,
 * [B,H,d_v,d_k] float32.
 *   q, k [B,T,H,dk], v [B,T,H,dv], o [B,T,H,dv] contiguous (dtype); g [B,T,H] float32.
 *   S0 [B,H,dv,dk] float32 or NULL; ST [B,H,dv,dk] float32 or NULL. dk = dv = 128. */
size_t mira_gla_workspace_bytes(int B, int T, int H, int dk, int dv);
int mira_gla_chunked(const void *q, const void *k, const void *v, const float *g,
                     const float *S0, float *ST, void *o, int B, int T, int H, int dk, int dv,
                     int dtype, void *workspace, size_t workspace_bytes, void *stream);
/* One decode token: q, k [B,H,dk], v, o [B,H,dv], g [B,H]; S [B,H,dv,dk] updated in place. */
int mira_gla_step(const void *q, const void *k, const void *v, const float *g, float *S,
                  void *o, int B, int H, int dk, int dv, int dtype, void *stream);

/* ---------------------------------------------------------------------------------------------
 * The MiraBlock feed-forward's first projection and activation (model/mira_block.py:38-48,
 * down(SiLU(up(x)))): out[rows, out_features] = SiLU(x W^T + bias), bf16 in and out, as one
 * hipBLASLt GEMM whose epilogue adds the bias and applies SiLU before the single rounding.
 * x [rows, in_features], weight [out_features, in_features] (nn.Linear's layout), bias
 * [out_features], out [rows, out_features], all contiguous bf16. MIRA_DECLINE when hipBLASLt
 * offers no algorithm for the shape. The first call per shape and device sets up a plan (and
 * the first call per device a 32 MiB workspace); it is not for graph capture. */
int mira_linear_silu(const void *x, const void *weight, const void *bias, void *out,
                     long long rows, int in_features, int out_features, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MIRA_HIP_H */
