// The backward of the K-stage lattice scan: gradients of sum(dy * y) with respect to x, alpha,
// beta, rho, gamma, the write vectors s and the read vectors nu (what autograd returns through
// model/mira_mixer.py:246-387, and what the reference plugin's MatrixLatticeIIR.backward
// launches, kernel/cuda/mira_dspv2/mira.py:1295-1433).
//
// Per (b, c) the state V_t (K x M) has an adjoint lambda_t = dL/dV_t. With the token's levels
// level_k (k = 0..K, V_t = level_(0..K-1)) and e = dy SiLU(gamma), the adjoint of level_k is
//     Lambda_k = lambda_t[k] (k < K) + e rho_k nu_k,
// and the stages run backward (k = 1..K) from dU = Lambda_0:
//     d rs_k += Lambda_k U_in - dU V_(t-1)[k-1],   d rc_k += Lambda_k V_(t-1)[k-1] + dU U_in,
//     lambda_(t-1)[k-1] = rc_k Lambda_k - rs_k dU,  dU <- rs_k Lambda_k + rc_k dU,
// ending at dU = d(x s). A masked token passes lambda through and has zero gradients. The
// adjoint recurrence lambda_(t-1) = A_t^T (lambda_t + injection) is affine like the forward's,
// so the token axis is cut into chunks the same way:
//   adjoint summary   per (b, chunk > 0, channel): the chunk's lambda from a zero adjoint at its
//                     end, walked backward (needs no forward state);
//   adjoint combine   per (b, c, m), serial over the chunks from the last: the adjoint at every
//                     chunk's end, lambda_end(j) = Phi_(j+1)^T lambda_end(j+1) + summary(j+1), with
//                     the forward summary's Phi;
//   backward replay   per (b, chunk, channel group): the chunk's states recomputed from the state
//                     entering it (the forward combine's output, kept by a forward run at this
//                     chunk length) into registers, then the walk backward with every gradient;
//   reduce            ds and dnu sum over channels: each replay block leaves its channel group's
//                     sums per (b, t), and one pass adds the groups (and applies SiLU' when the
//                     caller wants the gradient of the raw write).
// The chunk is short (<= 16 tokens) so that a lane keeps the states entering the tokens of its
// chunk in registers: all of them (<= 64 floats), or half of them in each of two passes over the
// chunk. Per-(token, channel) sums over a channel's lanes use DPP; per-(token, slot) sums over
// the channels of a block are first added across a 16-lane row's channels with DPP, then go
// through an LDS tile, double-buffered (one barrier a token) unless a single buffer (two
// barriers) lets another block share the CU.
#include "lattice_common.hpp"
#include "mira_abi_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace mira {
namespace {

constexpr int BLOCK = 256;

// lanes per channel: a lane's share of one K x M state is at most 8 floats
__host__ __device__ constexpr int back_lanes(int K, int M) {
    int L = 1;
    while (K * M / L > 8 && L < M && L < 64) L *= 2;
    return L;
}

// tokens per chunk: the states of a chunk fit 128 registers a lane, and the staged
// per-(token, channel) quantities of a block fit 32 KiB of LDS
__host__ __device__ constexpr int back_chunk_for(int K, int M) {
    const int L = back_lanes(K, M), MV = M / L, G = BLOCK / L;
    int S = 16;
    while (S > 1 && (S * K * MV > 128 || S * G * (3 * K + 2) > 8192)) S /= 2;
    return S;
}

// lanes per channel in the adjoint summary: it keeps only the adjoint and sums nothing over lanes,
// so a lane may hold up to 16 floats of it, and a block takes up to 64 channels while their staged
// per-(token, channel) quantities fit 32 KiB: the block's read vectors, staged once, then serve
// more channels (32 floats a lane at K2 d_m 64 took 129 VGPRs, three waves a SIMD, and lost)
__host__ __device__ constexpr int summary_lanes(int K, int M) {
    const int S = back_chunk_for(K, M);
    int L = back_lanes(K, M);
    while (L > 1 && K * M / (L / 2) <= 16 && BLOCK / (L / 2) <= 64 &&
           S * (3 * K + 1) * (BLOCK / (L / 2)) * 4 <= 32768)
        L /= 2;
    return L;
}

// the (K, d_m) with backward kernels: the reference plugin's ORDER_MEMORIES
// (kernel/cuda/mira_dspv2/mira.py:185-190)
__host__ __device__ constexpr bool backward_serves(int K, int M) {
    return ((K == 1 || K == 8) && (M == 8 || M == 16)) ||
           ((K == 2 || K == 4) && (M == 8 || M == 16 || M == 32 || M == 64));
}

// cos, sin, r of a stage and their derivatives d cos/d alpha, d sin/d alpha, d r/d beta (the
// derivatives of model/mira_mixer.py:56-145 as autograd forms them; the rational maps switch to
// 1/alpha above |alpha| = 1 so nothing overflows).
__device__ __forceinline__ void stage_derivatives(float alpha, float beta, int radius_kind,
                                                  int rotation_kind, float &c, float &s, float &r,
                                                  float &dc, float &ds, float &dr) {
    if (rotation_kind == MOBIUS) {
        const bool small = fabsf(alpha) <= 1.0f;
        const float q = small ? alpha : rcp_refined(alpha);
        const float q2 = q * q;
        const float inv = rcp_refined(1.0f + q2);
        c = 2.0f * q * inv;
        s = (small ? (1.0f - q2) : (q2 - 1.0f)) * inv;
        // d cos = 2 (1 - a^2) / (1 + a^2)^2 = 2 q^2 (q^2 - 1) / (1 + q^2)^2 with q = 1/a;
        // d sin = -4 a / (1 + a^2)^2 = -4 q^3 / (1 + q^2)^2
        const float inv2 = inv * inv;
        dc = small ? 2.0f * (1.0f - q2) * inv2 : 2.0f * q2 * (q2 - 1.0f) * inv2;
        ds = small ? -4.0f * q * inv2 : -4.0f * q2 * q * inv2;
    } else if (rotation_kind == HYPERBOLIC) {
        const float e = exp_refined(-fabsf(alpha));
        const float inv = rcp_refined(fmaf(e, e, 1.0f));
        c = 2.0f * e * inv;
        s = copysignf(fmaf(-e, e, 1.0f) * inv, alpha);
        dc = -c * s;
        ds = c * c;
    } else {
        sincosf(alpha, &s, &c);
        dc = -s;
        ds = c;
    }
    if (radius_kind == CAUCHY) {
        r = rcp_refined(fmaf(beta, beta, 1.0f));
        dr = -2.0f * beta * r * r;
    } else if (radius_kind == GAUSSIAN) {
        r = exp_refined(-(beta * beta));
        dr = -2.0f * beta * r;
    } else if (radius_kind == EXPEXP) {
        const float inner = exp_refined(fminf(beta, 80.0f));
        r = exp_refined(-inner);
        dr = beta <= 80.0f ? -inner * r : 0.0f;
    } else if (radius_kind == EXPSOFTPLUS) {
        r = rcp_refined(1.0f + exp_refined(beta));
        dr = -r * (1.0f - r);
    } else {
        const float q = beta * beta;
        const float inv = rcp_refined(1.0f + q);
        r = q > 1.0f ? 1.0f - inv : q * inv;
        dr = 2.0f * beta * inv * inv;
    }
}

__device__ __forceinline__ float silu_slope(float g) {
    const float sigma = 1.0f / (1.0f + expf(-g));
    return sigma * (1.0f + g * (1.0f - sigma));
}

// Stage a chunk's per-(token, channel) quantities, [token][quantity][channel]:
// rc[K], rs[K], e rho[K+1] (e = dy SiLU(gamma)) and, with X, x. MODE is the stage mode when the
// kernel is built for one stage map, 0 when it reads a.mode.
template <typename IO, int K, bool X, int MODE>
__device__ __forceinline__ void stage_adjoint_tile(const LatticeBackArgs &a, int b, int first,
                                                   int n, int c0, int G, float *tc,
                                                   unsigned char *valid) {
    constexpr int NQ = 3 * K + 1 + (X ? 1 : 0);
    const int mode = MODE ? MODE : a.mode;
    const int radius_kind = radius_of(mode), rotation_kind = rotation_of(mode);
    for (int i = threadIdx.x; i < n * G; i += BLOCK) {
        const int tt = i / G, cl = i % G, c = c0 + cl;
        if (c >= a.C) continue;
        float *dst = tc + tt * NQ * G + cl;
        const long long row = (long long)b * a.T + first + tt;
        const IO *alpha = static_cast<const IO *>(a.alpha) + row * a.alpha_row + (long long)c * K;
        const IO *beta = static_cast<const IO *>(a.beta) + row * a.beta_row + (long long)c * K;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float rc, rs;
            stage_coefficients(load(alpha + k), load(beta + k), radius_kind, rotation_kind, rc, rs);
            dst[k * G] = rc;
            dst[(K + k) * G] = rs;
        }
        const float e = load(static_cast<const IO *>(a.grad_out) + row * a.C + c) *
                        silu(load(static_cast<const IO *>(a.gamma) + row * a.gamma_row + c));
        const IO *rho = static_cast<const IO *>(a.rho) + row * a.rho_row + (long long)c * (K + 1);
#pragma unroll
        for (int k = 0; k <= K; ++k) dst[(2 * K + k) * G] = e * load(rho + k);
        if constexpr (X) dst[(3 * K + 1) * G] = load(static_cast<const IO *>(a.x) + row * a.x_row + c);
    }
    for (int tt = threadIdx.x; tt < n; tt += BLOCK)
        valid[tt] = a.valid ? a.valid[(long long)b * a.T + first + tt] : 1;
}

// ---------------------------------------------------------------------------------------------
// adjoint summary: lambda at the start of chunk j > 0 from a zero adjoint at its end
// ---------------------------------------------------------------------------------------------
template <typename IO, int K, int M, int MODE>
__global__ __launch_bounds__(BLOCK) void lattice_adjoint_summary(LatticeBackArgs a) {
    constexpr int L = summary_lanes(K, M), G = BLOCK / L, MV = M / L;
    constexpr int S = back_chunk_for(K, M);
    constexpr int NQ = 3 * K + 1;
    constexpr int NR = (K + 1) * M;
    const int groups = (a.C + G - 1) / G;
    int block = blockIdx.x;
    const int group = block % groups;
    block /= groups;
    const int j = 1 + block % (a.chunks - 1);
    const int b = block / (a.chunks - 1);
    const int lane = threadIdx.x % L, cl = threadIdx.x / L, c = group * G + cl;
    const int first = j * a.chunk, n = min(a.chunk, a.T - first);

    __shared__ float s_nu[S * NR];
    __shared__ float s_tc[S * NQ * G];
    __shared__ unsigned char s_valid[S];
    const IO *read = static_cast<const IO *>(a.read);
    for (int i = threadIdx.x; i < n * NR; i += BLOCK) {
        const int tt = i / NR, rest = i % NR;
        s_nu[i] = load(read + ((long long)b * a.T + first + tt) * a.read_row + rest);
    }
    stage_adjoint_tile<IO, K, false, MODE>(a, b, first, n, group * G, G, s_tc, s_valid);
    __syncthreads();
    if (c >= a.C) return;
    float lam[K][MV];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int v = 0; v < MV; ++v) lam[k][v] = 0.0f;
    for (int t = n - 1; t >= 0; --t) {
        if (!s_valid[t]) continue;
        const float *q = s_tc + t * NQ * G + cl;
        float rc[K], rs[K], er[K + 1];
#pragma unroll
        for (int k = 0; k < K; ++k) { rc[k] = q[k * G]; rs[k] = q[(K + k) * G]; }
#pragma unroll
        for (int k = 0; k <= K; ++k) er[k] = q[(2 * K + k) * G];
        const float *nu = s_nu + t * NR;
#pragma unroll
        for (int v = 0; v < MV; ++v) {
            const int m = slot<M, L>(lane, v);
            float Lam[K + 1];
#pragma unroll
            for (int k = 0; k <= K; ++k) Lam[k] = fmaf(er[k], nu[k * M + m], k < K ? lam[k][v] : 0.0f);
            float dU = Lam[0];
#pragma unroll
            for (int k = 1; k <= K; ++k) {
                const float next = fmaf(rc[k - 1], Lam[k], -(rs[k - 1] * dU));
                dU = fmaf(rs[k - 1], Lam[k], rc[k - 1] * dU);
                lam[k - 1][v] = next;
            }
        }
    }
    const long long plane = ((long long)b * a.chunks + j) * a.C + c;
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int v = 0; v < MV; ++v) a.adjoint[(plane * K + k) * M + slot<M, L>(lane, v)] = lam[k][v];
}

// ---------------------------------------------------------------------------------------------
// adjoint combine: the adjoint at the end of every chunk, serial over the chunks from the last
// ---------------------------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(BLOCK) void lattice_adjoint_combine(LatticeBackArgs a) {
    const long long index = (long long)blockIdx.x * BLOCK + threadIdx.x;
    const long long total = (long long)a.B * a.C * a.M;
    if (index >= total) return;
    const int m = index % a.M;
    const int c = (index / a.M) % a.C;
    const int b = index / ((long long)a.M * a.C);
    // chunk j's adjoint summary and transition do not depend on the running adjoint, so they
    // are loaded D chunks at a time ahead of the serial chain (a wait on memory once per D
    // chunks, not once per chunk)
    constexpr int D = 8;
    const long long plane0 = (long long)b * a.chunks * a.C + c;   // chunk 0's plane
    const long long stride = (long long)a.C;                      // planes per chunk
    const int last = a.chunks - 1;
    float run[K];
#pragma unroll
    for (int k = 0; k < K; ++k) run[k] = 0.0f;
    for (int j0 = last; j0 >= 0; j0 -= D) {
        float summary[D][K], transition[D][K * K];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int j = j0 - d;
            const long long plane = plane0 + j * stride;
#pragma unroll
            for (int k = 0; k < K; ++k)
                summary[d][k] = j > 0 ? a.adjoint[(plane * K + k) * a.M + m] : 0.0f;
#pragma unroll
            for (int q = 0; q < K * K; ++q)
                transition[d][q] = (j > 0 && j < last) ? a.phi[plane * K * K + q] : 0.0f;
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int j = j0 - d;
            if (j >= 0) {
                const long long plane = plane0 + j * stride;
#pragma unroll
                for (int k = 0; k < K; ++k) a.adjoint[(plane * K + k) * a.M + m] = run[k];   // j's end
                // at the last chunk run is zero, and so is Phi^T run
                float next[K];
#pragma unroll
                for (int jj = 0; jj < K; ++jj) {
                    float value = summary[d][jj];
#pragma unroll
                    for (int i = 0; i < K; ++i) value = fmaf(transition[d][i * K + jj], run[i], value);
                    next[jj] = value;
                }
#pragma unroll
                for (int k = 0; k < K; ++k) run[k] = next[k];
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// backward replay: one chunk of one channel group, every gradient
// ---------------------------------------------------------------------------------------------
template <typename IO, int K, int M, int MODE>
__global__ __launch_bounds__(BLOCK) void lattice_backward_replay(LatticeBackArgs a) {
    constexpr int L = back_lanes(K, M), G = BLOCK / L, MV = M / L;
    constexpr int S = back_chunk_for(K, M);
    constexpr int NQ = 3 * K + 2;           // staged rc[K], rs[K], e rho[K+1], x;
                                            // then the sums d rc[K], d rs[K], P[K+1], dx
    constexpr int NS = (K + 2) * M;         // s, nu_0 .. nu_K of a token
    constexpr int NO = (K + 2) * M;         // per-token channel sums: ds, dnu_0 .. dnu_K
    // rows of partial channel sums a token leaves in LDS: a 16-lane row first adds its channels
    // with DPP (narrow channels), so one row of 16 lanes, or one wide channel, writes each set
    constexpr int RG = L < 16 ? BLOCK / 16 : G;
    constexpr int TPO = (BLOCK / NO >= RG) ? RG : (BLOCK / NO >= 1 ? BLOCK / NO : 1);
    constexpr int TPO2 = (TPO >= 32) ? 32 : (TPO >= 16) ? 16 : (TPO >= 8) ? 8 : (TPO >= 4) ? 4
                                                            : (TPO >= 2) ? 2 : 1;
    constexpr int PER_PASS = BLOCK / TPO2;
    constexpr int P = S * K * MV > 64 ? 2 : 1;   // passes over the chunk (S is a power of two)
    constexpr int SP = S / P;
    // the channel sums are double-buffered by token parity (one barrier a token) unless a single
    // buffer and a second barrier let more blocks share a CU's 160 KiB of LDS
    constexpr int LDS_ONE = (S * NS + S * NQ * G + RG * NO) * 4 + S;
    constexpr int LDS_TWO = LDS_ONE + RG * NO * 4;
    constexpr int RED_BUFFERS = 163840 / LDS_ONE > 163840 / LDS_TWO ? 1 : 2;
    static_assert(LDS_ONE + (RED_BUFFERS - 1) * RG * NO * 4 <= 65536, "LDS budget");
    int block = blockIdx.x;
    const int group = block % a.groups;
    block /= a.groups;
    const int j = block % a.chunks;
    const int b = block / a.chunks;
    const int lane = threadIdx.x % L, cl = threadIdx.x / L, c = group * G + cl;
    const bool active = c < a.C;
    const int first = j * a.chunk, n = min(a.chunk, a.T - first);

    __shared__ float s_sn[S * NS];
    __shared__ float s_tc[S * NQ * G];
    __shared__ __align__(16) float s_red[RED_BUFFERS][RG * NO];
    __shared__ unsigned char s_valid[S];
    const IO *write = static_cast<const IO *>(a.write);
    const IO *read = static_cast<const IO *>(a.read);
    for (int i = threadIdx.x; i < n * NS; i += BLOCK) {
        const int tt = i / NS, rest = i % NS;
        const long long row = (long long)b * a.T + first + tt;
        s_sn[i] = rest < M ? load(write + row * M + rest) : load(read + row * a.read_row + (rest - M));
    }
    stage_adjoint_tile<IO, K, true, MODE>(a, b, first, n, group * G, G, s_tc, s_valid);

    // the state entering the chunk and the adjoint at its end
    float V[K][MV], lam[K][MV];
    const long long plane = ((long long)b * a.chunks + j) * a.C + c;
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int v = 0; v < MV; ++v) {
            const int m = slot<M, L>(lane, v);
            float state = 0.0f, adjoint = 0.0f;
            if (active) {
                if (a.chunks > 1) {
                    state = a.entering[(plane * K + k) * M + m];
                    adjoint = a.adjoint[(plane * K + k) * M + m];
                } else if (a.state_in) {
                    state = a.state_in[(((long long)b * K + k) * a.C + c) * M + m];
                }
            }
            V[k][v] = state;
            lam[k][v] = adjoint;
        }
    __syncthreads();

    // The chunk goes backward in P passes of SP tokens, last pass first; each pass recomputes the
    // forward from the chunk's entering state and keeps the states entering its own SP tokens.
    // Two passes halve the registers of the kept states (S K MV = 128 floats at 16 tokens) for 8
    // more forward tokens a chunk.
    float V0[K][MV];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int v = 0; v < MV; ++v) V0[k][v] = V[k][v];
#pragma unroll
    for (int pass = P - 1; pass >= 0; --pass) {
        if (pass * SP >= n) continue;                                  // uniform over the block
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int v = 0; v < MV; ++v) V[k][v] = V0[k][v];
        // forward: the state entering every token of the pass
        float Vs[SP][K][MV];
#pragma unroll
        for (int t = 0; t < (pass + 1) * SP; ++t) {
            if (t >= pass * SP) {
#pragma unroll
                for (int k = 0; k < K; ++k)
#pragma unroll
                    for (int v = 0; v < MV; ++v) Vs[t - pass * SP][k][v] = V[k][v];
            }
            if (t < n && s_valid[t] && t + 1 < (pass + 1) * SP) {
                const float *q = s_tc + t * NQ * G + cl;
                float rc[K], rs[K];
#pragma unroll
                for (int k = 0; k < K; ++k) { rc[k] = q[k * G]; rs[k] = q[(K + k) * G]; }
                const float xv = q[(3 * K + 1) * G];
#pragma unroll
                for (int v = 0; v < MV; ++v) {
                    float U = xv * s_sn[t * NS + slot<M, L>(lane, v)];
#pragma unroll
                    for (int k = K; k >= 1; --k) {
                        const float delayed = V[k - 1][v];
                        const float level = fmaf(rc[k - 1], delayed, rs[k - 1] * U);
                        U = fmaf(rc[k - 1], U, -(rs[k - 1] * delayed));
                        if (k < K) V[k][v] = level;
                    }
                    V[0][v] = U;
                }
            }
        }

        // backward, token by token
#pragma unroll
        for (int t = (pass + 1) * SP - 1; t >= pass * SP; --t) {
            if (t >= n) continue;                                   // uniform over the block
            float sums[NQ];
            float red[K + 2][MV];
#pragma unroll
            for (int q = 0; q < NQ; ++q) sums[q] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < K + 2; ++kk)
#pragma unroll
                for (int v = 0; v < MV; ++v) red[kk][v] = 0.0f;
            if (s_valid[t]) {
                const float *q = s_tc + t * NQ * G + cl;
                float rc[K], rs[K], er[K + 1];
#pragma unroll
                for (int k = 0; k < K; ++k) { rc[k] = q[k * G]; rs[k] = q[(K + k) * G]; }
#pragma unroll
                for (int k = 0; k <= K; ++k) er[k] = q[(2 * K + k) * G];
                const float xv = q[(3 * K + 1) * G];
                const float *sw = s_sn + t * NS;
                const float *nu = sw + M;
#pragma unroll
                for (int v = 0; v < MV; ++v) {
                    const int m = slot<M, L>(lane, v);
                    const float sm = sw[m];
                    float Uin[K + 1], level[K + 1];
                    float U = xv * sm;
#pragma unroll
                    for (int k = K; k >= 1; --k) {
                        const float delayed = Vs[t - pass * SP][k - 1][v];
                        Uin[k] = U;
                        level[k] = fmaf(rc[k - 1], delayed, rs[k - 1] * U);
                        U = fmaf(rc[k - 1], U, -(rs[k - 1] * delayed));
                    }
                    level[0] = U;
                    float Lam[K + 1];
#pragma unroll
                    for (int k = 0; k <= K; ++k) {
                        const float nk = nu[k * M + m];
                        sums[2 * K + k] = fmaf(level[k], nk, sums[2 * K + k]);            // P_k
                        Lam[k] = fmaf(er[k], nk, k < K ? lam[k][v] : 0.0f);
                        red[1 + k][v] = er[k] * level[k];                               // dnu_k
                    }
                    float dU = Lam[0];
#pragma unroll
                    for (int k = 1; k <= K; ++k) {
                        const float delayed = Vs[t - pass * SP][k - 1][v];
                        sums[K + k - 1] = fmaf(Lam[k], Uin[k], fmaf(-dU, delayed, sums[K + k - 1]));
                        sums[k - 1] = fmaf(Lam[k], delayed, fmaf(dU, Uin[k], sums[k - 1]));
                        const float next = fmaf(rc[k - 1], Lam[k], -(rs[k - 1] * dU));
                        dU = fmaf(rs[k - 1], Lam[k], rc[k - 1] * dU);
                        lam[k - 1][v] = next;
                    }
                    sums[3 * K + 1] = fmaf(dU, sm, sums[3 * K + 1]);                     // dx
                    red[0][v] = dU * xv;                                                 // ds
                }
            }
            // per (token, channel): the sums over the channel's lanes replace the staged quantities
#pragma unroll
            for (int q = 0; q < NQ; ++q) sums[q] = lane_sum<L>(sums[q]);
            if (active && lane == 0) {
#pragma unroll
                for (int q = 0; q < NQ; ++q) s_tc[(t * NQ + q) * G + cl] = sums[q];
            }
            // per (token, slot): the channel group's sums -- a row's channels added with DPP, then
            // one set per row (or per wide channel) through LDS, double-buffered by token parity
            float *red_buffer = s_red[t % RED_BUFFERS];
            const int rowgroup = L < 16 ? (int)threadIdx.x / 16 : cl;
            const bool writer = L < 16 ? ((int)threadIdx.x % 16) < L : true;
#pragma unroll
            for (int kk = 0; kk < K + 2; ++kk) {
#pragma unroll
                for (int v = 0; v < MV; ++v) {
                    float value = active ? red[kk][v] : 0.0f;
                    if constexpr (L < 16) value = row_channel_sum<L>(value);
                    red[kk][v] = value;
                }
                if (writer) {
                    float *dst = red_buffer + rowgroup * NO + kk * M;
                    if constexpr (MV % 4 == 0) {
#pragma unroll
                        for (int v = 0; v < MV; v += 4)
                            *reinterpret_cast<float4 *>(dst + slot<M, L>(lane, v)) =
                                make_float4(red[kk][v], red[kk][v + 1], red[kk][v + 2], red[kk][v + 3]);
                    } else {
#pragma unroll
                        for (int v = 0; v < MV; ++v) dst[slot<M, L>(lane, v)] = red[kk][v];
                    }
                }
            }
            __syncthreads();
            const long long out_row = ((long long)group * a.B + b) * a.T + first + t;
#pragma unroll
            for (int o0 = 0; o0 < NO; o0 += PER_PASS) {
                const int o = o0 + threadIdx.x / TPO2, part = threadIdx.x % TPO2;
                float total = 0.0f;
                if (o < NO)
                    for (int g = part; g < RG; g += TPO2) total += red_buffer[g * NO + o];
                total = group_sum<TPO2>(total);
                if (o < NO && part == 0) a.partial[out_row * NO + o] = total;
            }
            if constexpr (RED_BUFFERS == 1) __syncthreads();   // the next token's sums reuse the buffer
        }
    }

    // per (token, channel) gradients, one thread per pair
    const int mode = MODE ? MODE : a.mode;
    const int radius_kind = radius_of(mode), rotation_kind = rotation_of(mode);
    for (int i = threadIdx.x; i < n * G; i += BLOCK) {
        const int tt = i / G, q = i % G, ch = group * G + q;
        if (ch >= a.C) continue;
        const long long row = (long long)b * a.T + first + tt;
        const float *res = s_tc + tt * NQ * G + q;
        const bool on = s_valid[tt] != 0;
        const IO *alpha = static_cast<const IO *>(a.alpha) + row * a.alpha_row + (long long)ch * K;
        const IO *beta = static_cast<const IO *>(a.beta) + row * a.beta_row + (long long)ch * K;
        const IO *rho = static_cast<const IO *>(a.rho) + row * a.rho_row + (long long)ch * (K + 1);
        IO *grad_alpha = static_cast<IO *>(a.grad_alpha) + row * a.grad_alpha_row + (long long)ch * K;
        IO *grad_beta = static_cast<IO *>(a.grad_beta) + row * a.grad_beta_row + (long long)ch * K;
        IO *grad_rho = static_cast<IO *>(a.grad_rho) + row * a.grad_rho_row + (long long)ch * (K + 1);
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float ga = 0.0f, gb = 0.0f;
            if (on) {
                float cs, sn, r, dcs, dsn, dr;
                stage_derivatives(load(alpha + k), load(beta + k), radius_kind, rotation_kind,
                                  cs, sn, r, dcs, dsn, dr);
                const float drc = res[k * G], drs = res[(K + k) * G];
                ga = r * fmaf(drc, dcs, drs * dsn);
                gb = dr * fmaf(drc, cs, drs * sn);
            }
            grad_alpha[k] = from_float<IO>(ga);
            grad_beta[k] = from_float<IO>(gb);
        }
        const float dy = load(static_cast<const IO *>(a.grad_out) + row * a.C + ch);
        const float g = load(static_cast<const IO *>(a.gamma) + row * a.gamma_row + ch);
        const float e = dy * silu(g);
        float readout = 0.0f;
#pragma unroll
        for (int k = 0; k <= K; ++k) {
            const float P = on ? res[(2 * K + k) * G] : 0.0f;
            readout = fmaf(load(rho + k), P, readout);
            grad_rho[k] = from_float<IO>(e * P);
        }
        static_cast<IO *>(a.grad_gamma)[row * a.grad_gamma_row + ch] =
            from_float<IO>(on ? dy * silu_slope(g) * readout : 0.0f);
        static_cast<IO *>(a.grad_x)[row * a.grad_x_row + ch] =
            from_float<IO>(on ? res[(3 * K + 1) * G] : 0.0f);
    }
}

// ---------------------------------------------------------------------------------------------
// reduce: ds and dnu, the channel groups' sums added (ds through SiLU' of the raw write when
// the caller wants that gradient)
// ---------------------------------------------------------------------------------------------
template <typename IO>
__global__ __launch_bounds__(BLOCK) void lattice_backward_reduce(LatticeBackArgs a) {
    // a thread takes four consecutive sums (one 16-byte load a group; (K + 2) d_m is a multiple
    // of four, so the four share a token and a quantity) and keeps eight groups' loads in flight;
    // each sum still adds the groups in order from zero
    constexpr int AHEAD = 8;
    const int NO = (a.K + 2) * a.M;
    const long long index = ((long long)blockIdx.x * BLOCK + threadIdx.x) * 4;
    const long long per_group = (long long)a.B * a.T * NO;
    if (index >= per_group) return;
    const float4 *part = reinterpret_cast<const float4 *>(a.partial + index);
    const long long stride = per_group / 4;
    float total[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int g = 0;
    for (; g + AHEAD <= a.groups; g += AHEAD) {
        float4 v[AHEAD];
#pragma unroll
        for (int u = 0; u < AHEAD; ++u) v[u] = part[(g + u) * stride];
#pragma unroll
        for (int u = 0; u < AHEAD; ++u) {
            total[0] += v[u].x; total[1] += v[u].y; total[2] += v[u].z; total[3] += v[u].w;
        }
    }
    for (; g < a.groups; ++g) {
        const float4 v = part[g * stride];
        total[0] += v.x; total[1] += v.y; total[2] += v.z; total[3] += v.w;
    }
    const long long row = index / NO;
    const int o = index % NO;
    const int kk = o / a.M, m = o % a.M;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (kk == 0) {
            if (a.raw_write)
                total[e] *= silu_slope(load(static_cast<const IO *>(a.raw_write) + row * a.raw_write_row + m + e));
            static_cast<IO *>(a.grad_write)[row * a.grad_write_row + m + e] = from_float<IO>(total[e]);
        } else {
            static_cast<IO *>(a.grad_read)[row * a.grad_read_row + (kk - 1) * a.M + m + e] =
                from_float<IO>(total[e]);
        }
    }
}

template <typename IO, int K, int M, int MODE>
int launch_backward(LatticeBackArgs &a, hipStream_t stream) {
    constexpr int G = BLOCK / back_lanes(K, M);
    if (a.chunk != back_chunk_for(K, M))
        return fail(MIRA_ERR_ARG, "mira: the backward needs the forward run at "
                                  "mira_lattice_backward_chunk's chunk length");
    a.groups = (a.C + G - 1) / G;
    if (a.chunks > 1) {
        constexpr int GS = BLOCK / summary_lanes(K, M);
        const long long blocks = (long long)a.B * (a.chunks - 1) * ((a.C + GS - 1) / GS);
        hipLaunchKernelGGL((lattice_adjoint_summary<IO, K, M, MODE>), dim3(blocks), dim3(BLOCK), 0,
                           stream, a);
        if (int rc = check_launch("lattice_adjoint_summary")) return rc;
        const long long threads = (long long)a.B * a.C * M;
        hipLaunchKernelGGL((lattice_adjoint_combine<K>), dim3((threads + BLOCK - 1) / BLOCK),
                           dim3(BLOCK), 0, stream, a);
        if (int rc = check_launch("lattice_adjoint_combine")) return rc;
    }
    const long long blocks = (long long)a.B * a.chunks * a.groups;
    hipLaunchKernelGGL((lattice_backward_replay<IO, K, M, MODE>), dim3(blocks), dim3(BLOCK), 0, stream, a);
    if (int rc = check_launch("lattice_backward_replay")) return rc;
    static_assert((K + 2) * M % 4 == 0, "the reduce takes four sums a thread");
    const long long threads = (long long)a.B * a.T * (K + 2) * M / 4;
    hipLaunchKernelGGL((lattice_backward_reduce<IO>), dim3((threads + BLOCK - 1) / BLOCK),
                       dim3(BLOCK), 0, stream, a);
    return check_launch("lattice_backward_reduce");
}

// bf16 at the mixer's two geometries (K 2 with d_m 16 and 64) runs backward kernels built for
// their one stage map, as the forward does; everything else reads the map at run time
template <typename IO, int K, int M>
int backward_map(LatticeBackArgs &a, hipStream_t s) {
    if constexpr (std::is_same<IO, bf16_t>::value && K == 2 && (M == 16 || M == 64)) {
        switch (a.mode) {
            case 3: return launch_backward<IO, K, M, 3>(a, s);
            case 6: return launch_backward<IO, K, M, 6>(a, s);
            case 7: return launch_backward<IO, K, M, 7>(a, s);
            case 8: return launch_backward<IO, K, M, 8>(a, s);
            case 9: return launch_backward<IO, K, M, 9>(a, s);
            case 10: return launch_backward<IO, K, M, 10>(a, s);
            case 11: return launch_backward<IO, K, M, 11>(a, s);
            case 12: return launch_backward<IO, K, M, 12>(a, s);
            case 13: return launch_backward<IO, K, M, 13>(a, s);
            case 14: return launch_backward<IO, K, M, 14>(a, s);
            case 15: return launch_backward<IO, K, M, 15>(a, s);
            case 16: return launch_backward<IO, K, M, 16>(a, s);
            case 17: return launch_backward<IO, K, M, 17>(a, s);
            case 18: return launch_backward<IO, K, M, 18>(a, s);
            case 19: return launch_backward<IO, K, M, 19>(a, s);
        }
    }
    return launch_backward<IO, K, M, 0>(a, s);
}

template <typename IO, int K>
int backward_m(LatticeBackArgs &a, hipStream_t s) {
    switch (a.M) {
        case 8: return backward_map<IO, K, 8>(a, s);
        case 16: return backward_map<IO, K, 16>(a, s);
        case 32: if constexpr (backward_serves(K, 32)) return backward_map<IO, K, 32>(a, s); break;
        case 64: if constexpr (backward_serves(K, 64)) return backward_map<IO, K, 64>(a, s); break;
    }
    return fail(MIRA_DECLINE, "mira: no backward kernel for this d_m");
}

template <typename IO>
int backward_k(LatticeBackArgs &a, hipStream_t s) {
    switch (a.K) {
        case 1: return backward_m<IO, 1>(a, s);
        case 2: return backward_m<IO, 2>(a, s);
        case 4: return backward_m<IO, 4>(a, s);
        case 8: return backward_m<IO, 8>(a, s);
    }
    return fail(MIRA_DECLINE, "mira: no backward kernel for this order");
}

}  // namespace

int lattice_backward_chunk(int K, int M) {
    if (!backward_serves(K, M)) return 0;
    return back_chunk_for(K, M);
}

size_t lattice_backward_workspace(int B, int T, int C, int K, int M) {
    const int S = lattice_backward_chunk(K, M);
    if (!S) return 0;
    const int G = BLOCK / back_lanes(K, M);
    const long long chunks = (T + S - 1) / S;
    const long long groups = (C + G - 1) / G;
    const long long adjoint = chunks > 1 ? (long long)B * chunks * C * K * M : 0;
    const long long partial = groups * B * T * (K + 2) * M;
    return (size_t)(adjoint + partial) * sizeof(float);
}

int lattice_backward_launch(LatticeBackArgs &a, hipStream_t stream) {
    switch (a.dtype) {
        case MIRA_F32: return backward_k<float>(a, stream);
        case MIRA_BF16: return backward_k<bf16_t>(a, stream);
        case MIRA_F16: return backward_k<f16_t>(a, stream);
    }
    return fail(MIRA_DECLINE, "mira: unsupported dtype");
}

}  // namespace mira
