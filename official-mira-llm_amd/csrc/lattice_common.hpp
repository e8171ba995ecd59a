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

// DPP lane movement within a 16-lane row.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                              0xf, 0xf, false));
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

}  // namespace mira
