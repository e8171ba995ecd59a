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

// Sum over the L lanes of a channel group (adjacent lanes): cross-lane DPP within a quad,
// then butterflies through the LDS crossbar for wider groups.
template <int L>
__device__ __forceinline__ float lane_sum(float v) {
    if constexpr (L >= 2)
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                0xB1, 0xf, 0xf, false));
    if constexpr (L >= 4)
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                0x4E, 0xf, 0xf, false));
#pragma unroll
    for (int offset = 4; offset < L; offset <<= 1) v += __shfl_xor(v, offset, 64);
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

}  // namespace mira
