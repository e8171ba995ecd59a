// Pieces of the lattice scan shared by the replay (lattice.hip) and the scan that forms its own
// coefficients from the control (lattice_control.hip): how a channel's state is spread over lanes,
// the staged per-(token, channel) coefficient layout, and one token of the update and readout.
#pragma once
#include "mira_device.hpp"

namespace mira {

__host__ __device__ constexpr int lanes_for(int K, int M) {
    // the fewest lanes that keep a lane's share of the state at <= 32 floats
    int L = 1;
    while (K * M / L > 32 && L < M && L < 64) L *= 2;
    return L;
}

// Floats of per-(token, channel) coefficients staged per token: r cos and r sin of the K stages
// and x (summary), plus rho[K+1] and the SiLU gate (replay). Staged as [quantity][channel]:
// rc[K], rs[K], x, rho[K+1], gate.
__host__ __device__ constexpr int coef_count(int K, bool readout) {
    return readout ? 3 * K + 3 : 2 * K + 1;
}

// Memory slot of (lane, v): runs of four consecutive slots per lane (16-byte accesses) when a lane
// owns a multiple of four slots, lane-interleaved single slots otherwise.
template <int M, int L>
__device__ __forceinline__ int slot(int lane, int v) {
    constexpr int MV = M / L;
    if constexpr (MV % 4 == 0) return ((v >> 2) * L + lane) * 4 + (v & 3);
    else return v * L + lane;
}

// DPP lane movement within a 16-lane row. Every pattern used here reads a lane of the same row,
// so the bound-zero form changes nothing, and it lets the compiler fold the movement into the
// consuming add as its DPP operand.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xf, 0xf, true));
}

// Sum over the L lanes of a channel group (adjacent, aligned lanes), in every lane of the group:
// quad permutes for the first two steps, then the row's half-mirror (lane i <-> 7 - i) and mirror
// (i <-> 15 - i), which pair each quad or half-row with the other one of its group, all as DPP
// operands of the add; only groups wider than a row go through the LDS crossbar.
template <int L>
__device__ __forceinline__ float lane_sum(float v) {
    if constexpr (L >= 2) v += dpp<0xB1>(v);            // quad_perm [1,0,3,2]
    if constexpr (L >= 4) v += dpp<0x4E>(v);            // quad_perm [2,3,0,1]
    if constexpr (L >= 8) v += dpp<0x141>(v);           // row_half_mirror
    if constexpr (L >= 16) v += dpp<0x140>(v);          // row_mirror
#pragma unroll
    for (int offset = 16; offset < L; offset <<= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

// Sum over the channels of a 16-lane row whose channels are L lanes apart (L < 16), in every
// lane: row rotations by 8, 4, ... L, each the DPP operand of the add.
template <int L>
__device__ __forceinline__ float row_channel_sum(float v) {
    if constexpr (L < 16) v += dpp<0x128>(v);           // row_ror:8
    if constexpr (L < 8) v += dpp<0x124>(v);            // row_ror:4
    if constexpr (L < 4) v += dpp<0x122>(v);            // row_ror:2
    if constexpr (L < 2) v += dpp<0x121>(v);            // row_ror:1
    return v;
}

// One valid token of one channel on its L lanes: V (this lane's M/L slots of the K state rows)
// moves one step and the gated output comes back in every lane of the channel.
//   cf  the channel's coefficients, quantity q = cf(q): rc[K], rs[K], x, rho[K+1], gate
//   sw  the token's write vector s[M];  nu  its read vectors nu_0..nu_K, [K+1][M]
// Stage K's level rc_K V^(K-1) + rs_K x s is only read out, never kept: its sum over m is
// rc_K sum V^(K-1) nu_K + rs_K x sum s nu_K, so only U' is formed per slot (5K - 1 operations
// per slot instead of 5K + 2).
template <int K, int M, int L, typename Coefficient>
__device__ __forceinline__ float lattice_token(float (&V)[K][M / L], Coefficient cf,
                                               const float *sw, const float *nu, int lane) {
    constexpr int MV = M / L;
    float rc[K], rs[K], rho[K + 1];
#pragma unroll
    for (int k = 0; k < K; ++k) { rc[k] = cf(k); rs[k] = cf(K + k); }
    const float xv = cf(2 * K);
#pragma unroll
    for (int k = 0; k <= K; ++k) rho[k] = cf(2 * K + 1 + k);
    const float gate = cf(3 * K + 2);
    const float rcx = rc[K - 1] * xv;
    float acc[K + 1], sig = 0.0f;
#pragma unroll
    for (int k = 0; k <= K; ++k) acc[k] = 0.0f;
#pragma unroll
    for (int v = 0; v < MV; ++v) {
        const int m = slot<M, L>(lane, v);
        const float sv = sw[m];
        sig = fmaf(sv, nu[K * M + m], sig);
        acc[K] = fmaf(V[K - 1][v], nu[K * M + m], acc[K]);
        float U = fmaf(rcx, sv, -(rs[K - 1] * V[K - 1][v]));
#pragma unroll
        for (int k = K - 1; k >= 1; --k) {
            const float delayed = V[k - 1][v];
            const float up = rs[k - 1] * U, down = rs[k - 1] * delayed;
            V[k][v] = fmaf(rc[k - 1], delayed, up);        // level_k, kept
            U = fmaf(rc[k - 1], U, -down);
            acc[k] = fmaf(V[k][v], nu[k * M + m], acc[k]);
        }
        V[0][v] = U;
        acc[0] = fmaf(U, nu[m], acc[0]);
    }
    float y = rho[K] * fmaf(rc[K - 1], acc[K], rs[K - 1] * xv * sig);
#pragma unroll
    for (int k = 0; k < K; ++k) y = fmaf(rho[k], acc[k], y);
    return gate * lane_sum<L>(y);
}

// The replay's token in its scaled form (K <= 2). Each state row k is kept divided by a
// per-channel scale sigma_k (registers of every lane of the channel), chosen per token so that
// every output of the update is one fused multiply-add of two inputs with a unit coefficient on
// one of them:
//     U^  = V~_(K-1) + cu s                         (U = mu U^,  mu = -rs_(K-1) sigma_(K-1))
//     V~_1' = V~_0 + ta U^,  U^' = U^ + tb V~_0      (K = 2: sigma_1' = rc_0 sigma_0, mu' = rc_0 mu)
//     V~_0' = U^                                    (sigma_0' = mu')
// 3K + 1 operations per (t, c, m) with the readout (7 at K = 2) instead of 5K; the three
// coefficients cost a lane about a dozen operations per token. The caller multiplies the scales
// back into the state (scaled_renormalise) at least once per tile and wherever one falls below
// 2^-40. A coefficient that enters a scale is kept at least 2^-24 of its stage's larger
// coefficient and 2^-40 in magnitude (scale_factor), so with two such factors per token every
// scale stays a normal float. Staged quantities, q = cf(q), from stage_scaled_coefficients:
//     rc_0, rs_0 (K = 2: the rotation stage, rc_0 floored), rs_(K-1) floored, rc_(K-1) x,
//     gate rho_k (k < K), gate rho_K rc_(K-1), gate rho_K rs_(K-1) x.
__host__ __device__ constexpr int scaled_coef_count(int K) { return 3 * K + 2; }

__device__ __forceinline__ float scale_factor(float v, float stage_max) {
    const float floor = fmaxf(0x1p-24f * stage_max, 0x1p-40f);
    return fabsf(v) >= floor ? v : copysignf(floor, v);
}

// the staged quantities of one (token, channel) from its stage coefficients, x, rho and gate
template <int K>
__device__ __forceinline__ void stage_scaled_coefficients(float *dst, int G, const float (&rc)[K],
                                                          const float (&rs)[K], float x,
                                                          const float (&rho)[K + 1], float gate) {
    static_assert(K >= 1 && K <= 2, "the scaled token serves K <= 2");
    if constexpr (K == 2) {
        dst[0] = scale_factor(rc[0], fmaxf(fabsf(rc[0]), fabsf(rs[0])));
        dst[G] = rs[0];
    }
    dst[(2 * K - 2) * G] = scale_factor(rs[K - 1], fmaxf(fabsf(rc[K - 1]), fabsf(rs[K - 1])));
    dst[(2 * K - 1) * G] = rc[K - 1] * x;
#pragma unroll
    for (int k = 0; k < K; ++k) dst[(2 * K + k) * G] = gate * rho[k];
    dst[3 * K * G] = gate * rho[K] * rc[K - 1];
    dst[(3 * K + 1) * G] = gate * rho[K] * rs[K - 1] * x;
}

template <int K, int M, int L, typename Coefficient>
__device__ __forceinline__ float lattice_token_scaled(float (&V)[K][M / L], float (&sigma)[K],
                                                      Coefficient cf, const float *sw,
                                                      const float *nu, int lane) {
    static_assert(K >= 1 && K <= 2, "the scaled token serves K <= 2");
    constexpr int MV = M / L;
    float mu = -cf(2 * K - 2) * sigma[K - 1];
    const float cu = cf(2 * K - 1) * __builtin_amdgcn_rcpf(mu);
    float ta = 0.0f, tb = 0.0f, next1 = 0.0f;
    if constexpr (K == 2) {
        const float rc0 = cf(0), rs0 = cf(1);
        next1 = rc0 * sigma[0];
        ta = rs0 * mu * __builtin_amdgcn_rcpf(next1);
        const float mu_next = rc0 * mu;
        tb = -rs0 * sigma[0] * __builtin_amdgcn_rcpf(mu_next);
        mu = mu_next;
    }
    float acc[K + 1], sig = 0.0f;
#pragma unroll
    for (int k = 0; k <= K; ++k) acc[k] = 0.0f;
#pragma unroll
    for (int v = 0; v < MV; ++v) {
        const int m = slot<M, L>(lane, v);
        const float sv = sw[m];
        sig = fmaf(sv, nu[K * M + m], sig);
        acc[K] = fmaf(V[K - 1][v], nu[K * M + m], acc[K]);
        float U = fmaf(cu, sv, V[K - 1][v]);
        if constexpr (K == 2) {
            const float delayed = V[0][v];
            V[1][v] = fmaf(ta, U, delayed);
            U = fmaf(tb, delayed, U);
            acc[1] = fmaf(V[1][v], nu[M + m], acc[1]);
        }
        V[0][v] = U;
        acc[0] = fmaf(U, nu[m], acc[0]);
    }
    // readout weights: gate rho_k sigma_k' (k < K), gate rho_K rc_(K-1) sigma_(K-1), gate rho_K rs x
    float y = cf(3 * K + 1) * sig;
    y = fmaf(cf(3 * K) * sigma[K - 1], acc[K], y);
    y = fmaf(cf(2 * K) * mu, acc[0], y);
    if constexpr (K == 2) y = fmaf(cf(2 * K + 1) * next1, acc[1], y);
    sigma[0] = mu;
    if constexpr (K == 2) sigma[1] = next1;
    return lane_sum<L>(y);
}

// whether the scales must go back into the state after this token: below 2^-40
template <int K>
__device__ __forceinline__ bool scales_small(const float (&sigma)[K]) {
    bool small = false;
#pragma unroll
    for (int k = 0; k < K; ++k) small = small || fabsf(sigma[k]) < 0x1p-40f;
    return small;
}

template <int K, int MV>
__device__ __forceinline__ void scaled_renormalise(float (&V)[K][MV], float (&sigma)[K]) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int v = 0; v < MV; ++v) V[k][v] *= sigma[k];
        sigma[k] = 1.0f;
    }
}

}  // namespace mira
