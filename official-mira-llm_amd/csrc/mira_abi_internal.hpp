// Host-side plumbing shared by the kernel translation units and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "../../include/mira_hip.h"

namespace mira {

// Records the message returned by mira_last_error() on this thread and returns `code`.
int fail(int code, const std::string &message);

// Launch-status check after a kernel launch: MIRA_ERR_HIP with the HIP error string on failure.
int check_launch(const char *what);

// --- general lattice ------------------------------------------------------------------------
struct LatticeArgs {
    const void *x;       long long x_row;
    const void *alpha;   long long alpha_row;
    const void *beta;    long long beta_row;
    const void *rho;     long long rho_row;
    const void *gamma;   long long gamma_row;
    const void *write;                         // [B,T,M] contiguous
    const void *read;    long long read_row;   // [B,T,K+1,M], dense tail
    const uint8_t *valid;                      // [B,T] or null
    const float *state_in;                     // [B,K,C,M] or null
    float *state_out;                          // [B,K,C,M] or null
    void *out;                                 // [B,T,C] contiguous
    int B, T, C, K, M;
    int dtype, mode;
    int chunk, chunks;
    float *phi;                                // [B,chunks,C,K,K]
    float *carry;                              // [B,chunks,C,K,M]
    int carry_chunks, carry_step;              // the replay's view of the carries: planes per
                                               // sequence and per replay chunk (0: chunks, 1)
};
bool lattice_supported(int K, int M, int dtype);
int lattice_lanes(int K, int M);
int lattice_plan_chunk(int B, int T, int C, int K, int M);
size_t lattice_workspace(int B, int T, int C, int K, int M, int chunk);
int lattice_launch(LatticeArgs &a, hipStream_t stream);

// --- the lattice backward (gradients of the scan) --------------------------------------------
struct LatticeBackArgs {
    const void *x;       long long x_row;
    const void *alpha;   long long alpha_row;
    const void *beta;    long long beta_row;
    const void *rho;     long long rho_row;
    const void *gamma;   long long gamma_row;
    const void *write;                         // [B,T,M] contiguous
    const void *read;    long long read_row;   // [B,T,K+1,M], dense tail
    const uint8_t *valid;                      // [B,T] or null
    const float *state_in;                     // [B,K,C,M] or null (the forward's entering state)
    const void *grad_out;                      // [B,T,C] contiguous
    void *grad_x;        long long grad_x_row;
    void *grad_alpha;    long long grad_alpha_row;
    void *grad_beta;     long long grad_beta_row;
    void *grad_rho;      long long grad_rho_row;
    void *grad_gamma;    long long grad_gamma_row;
    void *grad_write;    long long grad_write_row;
    const void *raw_write; long long raw_write_row;   // or null: grad_write gets SiLU' of it
    void *grad_read;     long long grad_read_row;
    int B, T, C, K, M, dtype, mode;
    int chunk, chunks, groups;
    const float *phi;                          // forward workspace: [B,chunks,C,K,K]
    const float *entering;                     // forward workspace: [B,chunks,C,K,M]
    float *adjoint;                            // [B,chunks,C,K,M]
    float *partial;                            // [groups,B,T,K+2,M]
};
int lattice_backward_chunk(int K, int M);
size_t lattice_backward_workspace(int B, int T, int C, int K, int M);
int lattice_backward_launch(LatticeBackArgs &a, hipStream_t stream);

// --- the lattice scan forming its coefficients from the control ------------------------------
struct LatticeControlArgs {
    const void *x;        long long x_row;
    const void *control;                       // [B,T,R] contiguous
    const void *weight;   long long weight_row; // coefficient_projection weight, [rows, R]
    const void *bias;                          // [rows] or null
    long long alpha_first, beta_first, rho_first;   // rows of alpha(c=0,k=0), beta(0,0), rho(0,0)
    const void *gamma;    long long gamma_row;
    const void *write;                         // [B,T,M] contiguous
    const void *read;     long long read_row;  // [B,T,K+1,M], dense tail
    const uint8_t *valid;                      // [B,T] or null
    const float *state_in;                     // [B,K,C,M] or null
    float *state_out;                          // [B,K,C,M] or null
    void *out;                                 // [B,T,C] contiguous
    int B, T, C, K, M, R, mode;
};
bool lattice_control_serves(int B, int T, int C, int K, int M, int R, int dtype);
int lattice_control_launch(const LatticeControlArgs &a, hipStream_t stream);

// --- conv + diagonal scan -------------------------------------------------------------------
struct DiagArgs {
    const void *x;            // [B,T,D] contiguous
    const void *a;            // [B,T,D] contiguous
    const float *w;           // [D,W]
    const float *bias;        // [D] or null
    const float *h0;          // [B,D] or null
    const void *ring_in;      // [B,D,W-1] (x dtype) or null
    void *ring_out;           // [B,D,W-1] or null (may equal ring_in)
    long long pos;            // tokens absorbed before this call (ring slot origin)
    void *y;                  // [B,T,D]
    float *hT;                // [B,D] or null
    int B, T, D, W, dtype;
};
size_t diag_workspace(int B, int T, int D, int dtype);
int diag_scan_launch(const DiagArgs &a, void *workspace, size_t workspace_bytes,
                     hipStream_t stream);
int diag_step_launch(const DiagArgs &a, float *h, hipStream_t stream);
int diag_read_error(void *workspace, size_t workspace_bytes, unsigned *value);

// --- GLA matrix state -----------------------------------------------------------------------
struct GlaArgs {
    const void *q, *k, *v;    // [B,T,H,d] contiguous
    const float *g;           // [B,T,H]
    const float *S0;          // [B,H,dv,dk] or null
    float *ST;                // [B,H,dv,dk] or null (may equal S0)
    void *o;                  // [B,T,H,dv]
    int B, T, H, dk, dv, dtype;
};
int gla_step_launch(const GlaArgs &a, hipStream_t stream);
size_t gla_workspace(int B, int T, int H, int dk, int dv);
int gla_chunked_launch(const GlaArgs &a, void *workspace, size_t bytes, hipStream_t stream);
bool gla_chunk_applies(const GlaArgs &a);
int gla_chunk_launch(const GlaArgs &a, hipStream_t stream);

}  // namespace mira
