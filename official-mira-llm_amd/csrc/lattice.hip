// The K-stage matrix lattice scan (the reference operator, model/mira_mixer.py:246-387) on gfx950.
//
// Per (b, t, c) and memory slot m, with (rc_k, rs_k) = r_k (cos theta_k, sin theta_k):
//     U = x[b,t,c] s[b,t,m]
//     for k = K..1:  level_k = rs_k U + rc_k V^(k-1),   U = rc_k U - rs_k V^(k-1)
//     level_0 = U,   V^(0..K-1) <- level_(0..K-1)
//     y[b,t,c] = SiLU(gamma) sum_k rho_k sum_m level_k[m] nu_k[m]
// A masked token leaves V unchanged and writes 0.
//
// Work split (three launches when the token axis is cut, one when it is not):
//   summary  per (b, chunk, c): the chunk's affine map from a zero state -- Phi [K,K] (the K
//            basis states pushed through with zero input) and carry [K,M] (the state reached from
//            zero). The last chunk is never summarised: nothing reads it.
//   combine  per (b, c, m): S_(j+1) = Phi_j S_j + carry_j over the chunks, writing the state that
//            enters every chunk over its carry slot.
//   replay   per (b, chunk, c): the chunk from its entering state with the readout and the gate;
//            the last chunk stores the final state. A call cut finer than the planned chunk
//            length replays at the planned length from every step-th entering state. With one chunk this is the whole scan, and at
//            T = 1 it is the decode step. Stage K's level is never kept, so the replay reads it
//            out as rc_K sum_m V^(K-1) nu_K + rs_K x sum_m s nu_K instead of forming it per m:
//            5K - 1 operations per (t, c, m) instead of 5K + 2. At K <= 2, with a channel on
//            several lanes, the state rows are kept divided by per-channel scales that make every
//            update output one fused multiply-add (lattice_token_scaled): 3K + 1 operations.
// A block is 256 threads = G channels x L lanes; lane l of a channel owns M/L memory slots, so a
// channel's K x M state lives in registers. Per tile of TT tokens the block stages in LDS the
// write and read vectors s, nu (per (b, t), shared by every channel) and, per (token, channel),
// the stage coefficients r cos / r sin, x, rho and the gate: the stage maps are evaluated once per
// channel by one thread instead of by each of the channel's L lanes, and the tile's loads are
// issued together. Outputs of a tile leave through LDS as whole channel rows.
#include "lattice_common.hpp"
#include "mira_abi_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace mira {
namespace {

constexpr int BLOCK = 256;

__host__ __device__ constexpr int tile_for(int K, int M) {
    // tokens staged per LDS tile: s and nu <= 16 KiB, the coefficient tile <= 24 KiB, <= 8 tokens
    int t = 8;
    const int G = BLOCK / lanes_for(K, M);
    while (t > 1 && (t * (K + 2) * M * 4 > 16384 || t * coef_count(K, true) * G * 4 > 24576)) t /= 2;
    return t;
}

// Stage one token tile of a channel group: per (token, channel) the stage coefficients (once per
// channel, not once per lane), x, and for the readout rho and the gate; per token the valid flag.
// Layout coef[token][quantity][channel] so that a wave's reads of one quantity are contiguous.
// MODE is the stage mode when the kernel is built for one stage map, 0 when it reads a.mode.
// SCALED stages the scaled token's quantities (stage_scaled_coefficients) instead.
template <typename IO, int K, bool READOUT, int MODE = 0, bool SCALED = false>
__device__ __forceinline__ void stage_coefficient_tile(const LatticeArgs &a, int b, int tile, int n,
                                                       int c0, int G, float *coef,
                                                       unsigned char *valid) {
    constexpr int NC = coef_count(K, READOUT);
    const int mode = MODE ? MODE : a.mode;
    const int radius_kind = radius_of(mode), rotation_kind = rotation_of(mode);
    for (int i = threadIdx.x; i < n * G; i += BLOCK) {
        const int tt = i / G, cl = i % G, c = c0 + cl;
        float *dst = coef + tt * NC * G + cl;
        if (c >= a.C) continue;
        const long long row = (long long)b * a.T + tile + tt;
        const IO *alpha = static_cast<const IO *>(a.alpha) + row * a.alpha_row + (long long)c * K;
        const IO *beta = static_cast<const IO *>(a.beta) + row * a.beta_row + (long long)c * K;
        if constexpr (SCALED) {
            float rc[K], rs[K], rho_v[K + 1];
#pragma unroll
            for (int k = 0; k < K; ++k)
                stage_coefficients(load(alpha + k), load(beta + k), radius_kind, rotation_kind, rc[k], rs[k]);
            const IO *rho = static_cast<const IO *>(a.rho) + row * a.rho_row + (long long)c * (K + 1);
#pragma unroll
            for (int k = 0; k <= K; ++k) rho_v[k] = load(rho + k);
            stage_scaled_coefficients<K>(
                dst, G, rc, rs, load(static_cast<const IO *>(a.x) + row * a.x_row + c), rho_v,
                silu(load(static_cast<const IO *>(a.gamma) + row * a.gamma_row + c)));
            continue;
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float rc, rs;
            stage_coefficients(load(alpha + k), load(beta + k), radius_kind, rotation_kind, rc, rs);
            dst[k * G] = rc;
            dst[(K + k) * G] = rs;
        }
        dst[2 * K * G] = load(static_cast<const IO *>(a.x) + row * a.x_row + c);
        if constexpr (READOUT) {
            const IO *rho = static_cast<const IO *>(a.rho) + row * a.rho_row + (long long)c * (K + 1);
#pragma unroll
            for (int k = 0; k <= K; ++k) dst[(2 * K + 1 + k) * G] = load(rho + k);
            dst[(3 * K + 2) * G] = silu(load(static_cast<const IO *>(a.gamma) + row * a.gamma_row + c));
        }
    }
    for (int tt = threadIdx.x; tt < n; tt += BLOCK)
        valid[tt] = a.valid ? a.valid[(long long)b * a.T + tile + tt] : 1;
}

// ---------------------------------------------------------------------------------------------
// summary: Phi and carry of every chunk but the last, from a zero state
// ---------------------------------------------------------------------------------------------
template <typename IO, int K, int M, int MODE>
__global__ __launch_bounds__(BLOCK) void lattice_summary(LatticeArgs a) {
    constexpr int L = lanes_for(K, M);
    constexpr int G = BLOCK / L;
    constexpr int MV = M / L;
    constexpr int KB = (K + L - 1) / L;          // basis columns of Phi per lane
    constexpr int TT = tile_for(K, M);
    constexpr int NC = coef_count(K, false);
    const int groups = (a.C + G - 1) / G;
    const int summarised = a.chunks - 1;
    int block = blockIdx.x;
    const int group = block % groups;
    block /= groups;
    const int chunk_index = block % summarised;
    const int b = block / summarised;
    const int lane = threadIdx.x % L;
    const int cl = threadIdx.x / L;
    const int c = group * G + cl;
    const bool active = c < a.C;

    __shared__ float s_write[TT * M];
    __shared__ float s_coef[TT * NC * G];
    __shared__ unsigned char s_valid[TT];
    float V[K][MV];
    float P[K][KB];
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int v = 0; v < MV; ++v) V[k][v] = 0.0f;
#pragma unroll
        for (int i = 0; i < KB; ++i) P[k][i] = (lane + i * L == k) ? 1.0f : 0.0f;
    }
    const int first = chunk_index * a.chunk;
    const int last = min(first + a.chunk, a.T);
    const IO *write = static_cast<const IO *>(a.write);
    for (int tile = first; tile < last; tile += TT) {
        const int n = min(TT, last - tile);
        __syncthreads();
        for (int i = threadIdx.x; i < n * M; i += BLOCK)
            s_write[i] = load(write + ((long long)b * a.T + tile) * M + i);
        stage_coefficient_tile<IO, K, false, MODE>(a, b, tile, n, group * G, G, s_coef, s_valid);
        __syncthreads();
        if (!active) continue;
        for (int tt = 0; tt < n; ++tt) {
            if (!s_valid[tt]) continue;
            const float *cf = s_coef + tt * NC * G + cl;
            float rc[K], rs[K];
#pragma unroll
            for (int k = 0; k < K; ++k) { rc[k] = cf[k * G]; rs[k] = cf[(K + k) * G]; }
            const float xv = cf[2 * K * G];
#pragma unroll
            for (int v = 0; v < MV; ++v) {
                float U = xv * s_write[tt * M + slot<M, L>(lane, v)];
#pragma unroll
                for (int k = K; k >= 1; --k) {
                    const float delayed = V[k - 1][v];
                    const float level = fmaf(rc[k - 1], delayed, rs[k - 1] * U);
                    U = fmaf(rc[k - 1], U, -(rs[k - 1] * delayed));
                    if (k < K) V[k][v] = level;
                }
                V[0][v] = U;
            }
#pragma unroll
            for (int i = 0; i < KB; ++i) {
                float U = 0.0f;
#pragma unroll
                for (int k = K; k >= 1; --k) {
                    const float delayed = P[k - 1][i];
                    const float level = fmaf(rc[k - 1], delayed, rs[k - 1] * U);
                    U = fmaf(rc[k - 1], U, -(rs[k - 1] * delayed));
                    if (k < K) P[k][i] = level;
                }
                P[0][i] = U;
            }
        }
    }
    if (!active) return;
    const long long plane = ((long long)b * a.chunks + chunk_index) * a.C + c;
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int v = 0; v < MV; ++v) a.carry[(plane * K + k) * M + slot<M, L>(lane, v)] = V[k][v];
#pragma unroll
        for (int i = 0; i < KB; ++i) {
            const int j = lane + i * L;
            if (j < K) a.phi[(plane * K + k) * K + j] = P[k][i];
        }
    }
}

// ---------------------------------------------------------------------------------------------
// summary on the matrix cores (bf16 inputs): per channel the stage maps are affine in the state,
// V_t = A_t V_(t-1) + b_t U_t with U_t = x_t s_t[m], and A_t, b_t (K x K, K) do not depend on m.
// So the chunk's carry from a zero state is carry[k][m] = sum_s g_s[k] s_s[m] with
// g_s = A_L .. A_(s+1) b_s x_s, and Phi = A_L .. A_1: O(K^2) work per token instead of O(K M),
// and the sum over s is a GEMM,
//     carry[(c, k)][m] = sum_s g_s[c][k] . s_s[m],
// run on v_mfma_f32_32x32x16_bf16 with the left operand split into a bf16 high part and its
// rounding remainder (float32-level accuracy; s is bf16 already).
// A block owns 64 rows (c, k) -- 64 / K channels -- and walks the chunk backwards in tiles of 16
// tokens. Every lane is one token of the tile: a 16-lane row holds the tile's tokens for 64 / (16 K)
// channels, each lane computes its token's stage map, and the suffix products A_15 .. A_t of the
// tile come from a four-round scan across the row (DPP row shifts; lanes past the row's end read
// the identity). g_t = Pl A_15 .. A_(t+1) b_t x_t, where Pl is the product of the later tiles'
// maps, which every lane of the row carries (the tile's product is lane 0's inclusive scan).
// ---------------------------------------------------------------------------------------------
namespace summary_mfma {
constexpr int ROWS = 64, TT = 16, TP = TT + 8;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int drow(int lane, int i) { return 8 * (i >> 2) + ((lane >> 5) << 2) + (i & 3); }
__device__ __forceinline__ bf16x8 operand(const uint16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ uint16_t to_bf16(float v) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v)); }
__device__ __forceinline__ float from_bf16(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// lane i of a 16-lane row takes lane i + N's value; past the row's end it keeps `fill` (a zero
// fill is the DPP's own bound-zero mode, which needs no register holding the fill)
template <int N>
__device__ __forceinline__ float from_row_above(float v, float fill) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill),
                                                                 __builtin_bit_cast(int, v),
                                                                 0x100 + N, 0xf, 0xf, false));
}
template <int N>
__device__ __forceinline__ float from_row_above_or_zero(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 0x100 + N, 0xf, 0xf, true));
}
// X_t <- X_(t+N) X_t across the row (identity past its end): one round of the suffix scan
template <int N, int K>
__device__ __forceinline__ void suffix_round(float (&X)[K][K]) {
    float Y[K][K], Z[K][K];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int j = 0; j < K; ++j)
            Y[k][j] = k == j ? from_row_above<N>(X[k][j], 1.0f) : from_row_above_or_zero<N>(X[k][j]);
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int j = 0; j < K; ++j) {
            float v = Y[k][0] * X[0][j];
#pragma unroll
            for (int q = 1; q < K; ++q) v = fmaf(Y[k][q], X[q][j], v);
            Z[k][j] = v;
        }
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int j = 0; j < K; ++j) X[k][j] = Z[k][j];
}
}  // namespace summary_mfma

template <int K, int M, int MODE>
__global__ __launch_bounds__(BLOCK) void lattice_summary_mfma(LatticeArgs a) {
    using namespace summary_mfma;
    constexpr int G = ROWS / K;                  // channels per block
    constexpr int CP = G / TT;                   // channels per lane (16 rows of 16 token lanes)
    constexpr int CT = M / 32;                   // output column tiles
    constexpr int TILES = 2 * CT;                // 32 x 32 output tiles (2 row tiles)
    constexpr int PER_WAVE = (TILES + 3) / 4;
    constexpr int WPT = TT * M / BLOCK;          // s elements per thread per tile
    static_assert(BLOCK == 256 && CP >= 1 && CP * TT == G && WPT >= 1 && TT * M % BLOCK == 0,
                  "tile shape");
    const int groups = (a.C + G - 1) / G;
    const int summarised = a.chunks - 1;
    int block = blockIdx.x;
    const int group = block % groups;
    block /= groups;
    const int chunk_index = block % summarised;
    const int b = block / summarised;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int t = tid & (TT - 1), row = tid / TT;
    const int c0 = group * G, cr = c0 + row * CP;    // this lane's first channel
    const int mode = MODE ? MODE : a.mode;
    const int radius_kind = radius_of(mode), rotation_kind = rotation_of(mode);

    __shared__ alignas(16) uint16_t s_wT[M][TP];  // s^T of the tile, [m][token]
    __shared__ alignas(16) uint16_t s_hi[ROWS][TP], s_lo[ROWS][TP];   // g, [(c, k)][token]

    // raw inputs of this lane's token, loaded a tile ahead: alpha[K], beta[K], x per channel
    struct Raw { uint16_t al[CP][K], be[CP][K], x[CP], w[WPT]; bool on; };
    const uint16_t *alpha_p = static_cast<const uint16_t *>(a.alpha);
    const uint16_t *beta_p = static_cast<const uint16_t *>(a.beta);
    const uint16_t *x_p = static_cast<const uint16_t *>(a.x);
    const uint16_t *write = static_cast<const uint16_t *>(a.write);
    auto fetch = [&](Raw &r, int tile) {
        const long long rowi = (long long)b * a.T + tile + t;
        r.on = !a.valid || a.valid[rowi];
#pragma unroll
        for (int e = 0; e < CP; ++e) {
            const long long cc = cr + e < a.C ? cr + e : 0;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                r.al[e][k] = alpha_p[rowi * a.alpha_row + cc * K + k];
                r.be[e][k] = beta_p[rowi * a.beta_row + cc * K + k];
            }
            r.x[e] = x_p[rowi * a.x_row + cc];
        }
#pragma unroll
        for (int q = 0; q < WPT; ++q) {
            const int i = tid + q * BLOCK, tt = i / M, m = i % M;
            r.w[q] = write[((long long)b * a.T + tile + tt) * M + m];
        }
    };

    f32x16 acc[PER_WAVE];
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) acc[q] = f32x16{};
    // Pl: the product of the maps of the tiles after the current one (per channel of the lane);
    // after the last tile it is the chunk's Phi
    float Pl[CP][K][K];
#pragma unroll
    for (int e = 0; e < CP; ++e)
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int j = 0; j < K; ++j) Pl[e][k][j] = k == j ? 1.0f : 0.0f;

    const int first = chunk_index * a.chunk;
    const int last_tile = first + a.chunk - TT;
    Raw cur, next;
    fetch(cur, last_tile);
    for (int tile = last_tile; tile >= first; tile -= TT) {
        __syncthreads();                                       // previous tile's operands used
#pragma unroll
        for (int e = 0; e < CP; ++e) {
            // this token's stage map as an affine map of (V, U): A (K x K) and b, times x
            float X[K][K], bx[K];
            if (cur.on && cr + e < a.C) {
                float rc[K], rs[K];
#pragma unroll
                for (int k = 0; k < K; ++k)
                    stage_coefficients(from_bf16(cur.al[e][k]), from_bf16(cur.be[e][k]), radius_kind,
                                       rotation_kind, rc[k], rs[k]);
                const float xv = from_bf16(cur.x[e]);
#pragma unroll
                for (int col = 0; col <= K; ++col) {           // col < K: basis state e_col; K: U = 1
                    float V[K];
#pragma unroll
                    for (int k = 0; k < K; ++k) V[k] = (k == col) ? 1.0f : 0.0f;
                    float U = col == K ? 1.0f : 0.0f;
#pragma unroll
                    for (int k = K; k >= 1; --k) {
                        const float delayed = V[k - 1];
                        const float level = fmaf(rc[k - 1], delayed, rs[k - 1] * U);
                        U = fmaf(rc[k - 1], U, -(rs[k - 1] * delayed));
                        if (k < K) V[k] = level;
                    }
                    V[0] = U;
#pragma unroll
                    for (int k = 0; k < K; ++k) {
                        if (col < K) X[k][col] = V[k];
                        else bx[k] = V[k] * xv;
                    }
                }
            } else {                                           // masked or past C: V unchanged
#pragma unroll
                for (int k = 0; k < K; ++k) {
#pragma unroll
                    for (int j = 0; j < K; ++j) X[k][j] = k == j ? 1.0f : 0.0f;
                    bx[k] = 0.0f;
                }
            }
            // inclusive suffix products across the row: X_t = A_15 .. A_t
            suffix_round<1, K>(X);
            suffix_round<2, K>(X);
            suffix_round<4, K>(X);
            suffix_round<8, K>(X);
            // g_t = Pl A_15 .. A_(t+1) b_t x_t
            float zb[K];
#pragma unroll
            for (int k = 0; k < K; ++k) {
                float v = 0.0f;
#pragma unroll
                for (int j = 0; j < K; ++j)
                    v = fmaf(k == j ? from_row_above<1>(X[k][j], 1.0f) : from_row_above_or_zero<1>(X[k][j]),
                             bx[j], v);
                zb[k] = v;
            }
#pragma unroll
            for (int k = 0; k < K; ++k) {
                float g = 0.0f;
#pragma unroll
                for (int j = 0; j < K; ++j) g = fmaf(Pl[e][k][j], zb[j], g);
                const uint16_t hi = to_bf16(g);
                s_hi[(row * CP + e) * K + k][t] = hi;
                s_lo[(row * CP + e) * K + k][t] = to_bf16(g - from_bf16(hi));
            }
            // Pl <- Pl (A_15 .. A_0), the tile's product from lane 0 of the row
            float Tm[K][K], N[K][K];
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int j = 0; j < K; ++j) Tm[k][j] = __shfl(X[k][j], lane & ~(TT - 1));
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int j = 0; j < K; ++j) {
                    float v = Pl[e][k][0] * Tm[0][j];
#pragma unroll
                    for (int q = 1; q < K; ++q) v = fmaf(Pl[e][k][q], Tm[q][j], v);
                    N[k][j] = v;
                }
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int j = 0; j < K; ++j) Pl[e][k][j] = N[k][j];
        }
#pragma unroll
        for (int q = 0; q < WPT; ++q) {
            const int i = tid + q * BLOCK, tt = i / M, m = i % M;
            s_wT[m][tt] = cur.w[q];
        }
        if (tile - TT >= first) fetch(next, tile - TT);        // in flight during the GEMM
        __syncthreads();
        // carry += g[rows][tokens] . s[tokens][m]
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q) {
            const int tl = wave + 4 * q;
            if (TILES % 4 == 0 || tl < TILES) {
                const int rt = tl % 2, ct = tl / 2;
                const int kk = 8 * (lane >> 5);
                const bf16x8 B = operand(&s_wT[32 * ct + (lane & 31)][kk]);
                acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(operand(&s_hi[32 * rt + (lane & 31)][kk]), B,
                                                                 acc[q], 0, 0, 0);
                acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(operand(&s_lo[32 * rt + (lane & 31)][kk]), B,
                                                                 acc[q], 0, 0, 0);
            }
        }
        cur = next;
    }
    // carry rows (c, k) and Phi
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
        const int tl = wave + 4 * q;
        if (tl < TILES) {
            const int rt = tl % 2, ct = tl / 2;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = 32 * rt + drow(lane, i), m = 32 * ct + (lane & 31);
                const int c = c0 + r / K, k = r % K;
                if (c < a.C) {
                    const long long plane = ((long long)b * a.chunks + chunk_index) * a.C + c;
                    a.carry[(plane * K + k) * M + m] = acc[q][i];
                }
            }
        }
    }
    if (t == 0) {
#pragma unroll
        for (int e = 0; e < CP; ++e) {
            if (cr + e < a.C) {
                const long long plane = ((long long)b * a.chunks + chunk_index) * a.C + cr + e;
#pragma unroll
                for (int k = 0; k < K; ++k)
#pragma unroll
                    for (int j = 0; j < K; ++j) a.phi[(plane * K + k) * K + j] = Pl[e][k][j];
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// combine: the state entering every chunk, serial over the chunks of one (b, c, m)
// ---------------------------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(BLOCK) void lattice_combine(LatticeArgs a) {
    const long long index = (long long)blockIdx.x * BLOCK + threadIdx.x;
    const long long total = (long long)a.B * a.C * a.M;
    if (index >= total) return;
    const int m = index % a.M;
    const int c = (index / a.M) % a.C;
    const int b = index / ((long long)a.M * a.C);
    float S[K];
#pragma unroll
    for (int k = 0; k < K; ++k)
        S[k] = a.state_in ? a.state_in[(((long long)b * K + k) * a.C + c) * a.M + m] : 0.0f;
    // The chunk maps do not depend on the running state: they are loaded D chunks at a time
    // ahead of the serial chain, so a long chain (training runs 16-token chunks) waits on memory
    // once per D chunks instead of once per chunk.
    constexpr int D = 8;
    for (int j0 = 0; j0 < a.chunks; j0 += D) {
        float carry[D][K], phi[D][K * K];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int j = j0 + d;
            const bool summarised = j + 1 < a.chunks;
            const long long plane = ((long long)b * a.chunks + j) * a.C + c;
#pragma unroll
            for (int k = 0; k < K; ++k)
                carry[d][k] = summarised ? a.carry[(plane * K + k) * a.M + m] : 0.0f;
#pragma unroll
            for (int q = 0; q < K * K; ++q) phi[d][q] = summarised ? a.phi[plane * K * K + q] : 0.0f;
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int j = j0 + d;
            if (j < a.chunks) {
                const long long plane = ((long long)b * a.chunks + j) * a.C + c;
#pragma unroll
                for (int k = 0; k < K; ++k) a.carry[(plane * K + k) * a.M + m] = S[k];
                float next[K];
#pragma unroll
                for (int i = 0; i < K; ++i) {
                    float value = carry[d][i];
#pragma unroll
                    for (int jj = 0; jj < K; ++jj) value = fmaf(phi[d][i * K + jj], S[jj], value);
                    next[i] = value;
                }
#pragma unroll
                for (int k = 0; k < K; ++k) S[k] = next[k];
            }
        }
    }
}

// Four consecutive elements as floats, from an address aligned to four elements.
__device__ __forceinline__ float4 load4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ float4 load4(const bf16_t *p) {
    const uint2 w = *reinterpret_cast<const uint2 *>(p);
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
}
__device__ __forceinline__ float4 load4(const f16_t *p) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 h = *reinterpret_cast<const h4 *>(p);
    return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}

// `rows` rows of LEN elements, `stride` elements apart from `src`, into dst[row LEN + e] as
// floats: four elements a load and one 16-byte LDS store where `vector` says the rows start
// four-element aligned (the per-element loop cost the replay 16 VALU instructions an element)
template <typename IO, int LEN>
__device__ __forceinline__ void stage_rows(float *dst, const IO *src, long long stride, int rows,
                                           bool vector) {
    if (LEN % 4 == 0 && vector) {
        constexpr int Q = LEN / 4;
        for (int i = threadIdx.x; i < rows * Q; i += BLOCK) {
            const int r = i / Q, e = 4 * (i % Q);
            *reinterpret_cast<float4 *>(dst + r * LEN + e) = load4(src + r * stride + e);
        }
    } else {
        for (int i = threadIdx.x; i < rows * LEN; i += BLOCK) {
            const int r = i / LEN, e = i % LEN;
            dst[i] = load(src + r * stride + e);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// replay: the scan of one chunk from its entering state, with readout and gate
// ---------------------------------------------------------------------------------------------
// K <= 2 runs the scaled token where a channel spans several lanes
__host__ __device__ constexpr bool replay_scaled(int K, int M) { return K <= 2 && lanes_for(K, M) > 1; }

template <typename IO, int K, int M, int MODE>
__global__ __launch_bounds__(BLOCK) void lattice_replay(LatticeArgs a) {
    constexpr int L = lanes_for(K, M);
    constexpr int G = BLOCK / L;
    constexpr int MV = M / L;
    constexpr int TT = tile_for(K, M);
    constexpr int NC = coef_count(K, true);
    // K <= 2 runs the scaled token (one fused multiply-add per update output) where a channel
    // spans several lanes; a channel on one lane (K d_m <= 32) would hold the unrolled tile's
    // s and nu of every token in registers and keeps the direct form
    constexpr bool SCALED = replay_scaled(K, M);
    static_assert(!SCALED || scaled_coef_count(K) <= NC, "scaled coefficients fit the staged tile");
    const int groups = (a.C + G - 1) / G;
    int block = blockIdx.x;
    const int group = block % groups;
    block /= groups;
    const int chunk_index = block % a.chunks;
    const int b = block / a.chunks;
    const int lane = threadIdx.x % L;
    const int cl = threadIdx.x / L;
    const int c = group * G + cl;
    const bool active = c < a.C;

    __shared__ __align__(16) float s_write[TT * M];
    __shared__ __align__(16) float s_read[TT * (K + 1) * M];
    __shared__ float s_coef[TT * NC * G];
    __shared__ float s_out[TT * G];
    __shared__ unsigned char s_valid[TT];
    float V[K][MV];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int v = 0; v < MV; ++v) {
            float value = 0.0f;
            if (active) {
                const int m = slot<M, L>(lane, v);
                if (chunk_index > 0) {
                    const long long plane = (long long)b * (a.carry_chunks ? a.carry_chunks : a.chunks) +
                                            (long long)chunk_index * (a.carry_step ? a.carry_step : 1);
                    value = a.carry[((plane * a.C + c) * K + k) * M + m];
                }
                else if (a.state_in)
                    value = a.state_in[(((long long)b * K + k) * a.C + c) * M + m];
            }
            V[k][v] = value;
        }
    const int first = chunk_index * a.chunk;
    const int last = min(first + a.chunk, a.T);
    float sigma[K];                                            // the channel's scales (SCALED)
#pragma unroll
    for (int k = 0; k < K; ++k) sigma[k] = 1.0f;
    const IO *write = static_cast<const IO *>(a.write);
    const IO *read = static_cast<const IO *>(a.read);
    IO *out = static_cast<IO *>(a.out);
    const auto aligned4 = [](const void *p) {
        return (reinterpret_cast<uintptr_t>(p) & (4 * sizeof(IO) - 1)) == 0;
    };
    // four-element staging in the scaled replay of a compiled-in non-circular map only: the
    // direct-form kernels measured slower with it (K2 d_m 16 300 -> 421 us, K4 d_m 64 810 -> 907
    // us) and the circular maps' kernels went past 128 registers (K2 d_m 64 403 -> 498 us)
    constexpr bool CIRCULAR = MODE == 7 || (MODE >= 8 && (MODE - 8) % 3 == 2);
    const bool vector_rows = SCALED && MODE != 0 && !CIRCULAR && aligned4(write) &&
                             aligned4(read) && a.read_row % 4 == 0;
    for (int tile = first; tile < last; tile += TT) {
        const int n = min(TT, last - tile);
        __syncthreads();                                       // previous tile's outputs stored
        stage_rows<IO, M>(s_write, write + ((long long)b * a.T + tile) * M, M, n, vector_rows);
        stage_rows<IO, (K + 1) * M>(s_read, read + ((long long)b * a.T + tile) * a.read_row,
                                    a.read_row, n, vector_rows);
        stage_coefficient_tile<IO, K, true, MODE, SCALED>(a, b, tile, n, group * G, G, s_coef, s_valid);
        __syncthreads();
        // a full tile of live tokens runs unrolled without branches: the update's outputs then
        // rotate through registers instead of being copied back every token
        bool full = SCALED && n == TT;
        for (int tt = 0; tt < TT && full; ++tt) full = s_valid[tt] != 0;
        if (active && full) {
            if constexpr (SCALED) {
#pragma unroll
                for (int tt = 0; tt < TT; ++tt) {
                    const float *cf = s_coef + tt * NC * G + cl;
                    const float y = lattice_token_scaled<K, M, L>(
                        V, sigma, [&](int q) { return cf[q * G]; }, s_write + tt * M,
                        s_read + tt * (K + 1) * M, lane);
                    // the scales back into the state at the tile's end and where one runs small
                    if (tt == TT - 1 || scales_small(sigma)) scaled_renormalise(V, sigma);
                    if (lane == 0) s_out[tt * G + cl] = y;
                }
            }
        } else if (active) {
            for (int tt = 0; tt < n; ++tt) {
                float y = 0.0f;
                const float *cf = s_coef + tt * NC * G + cl;
                if (s_valid[tt]) {
                    if constexpr (SCALED)
                        y = lattice_token_scaled<K, M, L>(V, sigma, [&](int q) { return cf[q * G]; },
                                                          s_write + tt * M, s_read + tt * (K + 1) * M, lane);
                    else
                        y = lattice_token<K, M, L>(V, [&](int q) { return cf[q * G]; },
                                                   s_write + tt * M, s_read + tt * (K + 1) * M, lane);
                }
                if constexpr (SCALED) {
                    if (tt == n - 1 || scales_small(sigma)) scaled_renormalise(V, sigma);
                }
                if (lane == 0) s_out[tt * G + cl] = y;
            }
        }
        __syncthreads();                                       // the tile's outputs
        for (int i = threadIdx.x; i < n * G; i += BLOCK) {
            const int tt = i / G, cc = group * G + i % G;
            if (cc < a.C) out[((long long)b * a.T + tile + tt) * a.C + cc] = from_float<IO>(s_out[i]);
        }
    }
    if (active && a.state_out && chunk_index == a.chunks - 1) {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int v = 0; v < MV; ++v)
                a.state_out[(((long long)b * K + k) * a.C + c) * M + slot<M, L>(lane, v)] = V[k][v];
    }
}


// ---------------------------------------------------------------------------------------------
// decode step (T = 1): a stream of the state
// ---------------------------------------------------------------------------------------------
// One token moves the whole [B,K,C,M] float32 state through HBM once each way, so the step is a
// stream: a block takes one sequence b and 256 / (M/8) channels, a lane owns 8 consecutive memory
// slots of one channel (two 16-byte accesses per state row), s and nu of the sequence are staged
// in LDS once, and the stage maps run once per channel (see the kernel for the load order that
// keeps the state loads in flight meanwhile). The update and readout are the replay's (stage
// K's level read out through sum V^(K-1) nu_K and sum s nu_K). A masked token copies the state
// and writes 0.
__host__ __device__ constexpr bool step_kernel_serves(int K, int M) { return K <= 4 && M >= 8 && M <= 128; }

template <typename IO, int K, int M, bool HAS_STATE, int SB>
__global__ __launch_bounds__(SB) void lattice_step_kernel(LatticeArgs a) {
    constexpr int LPC = M / 8;                   // lanes of a channel
    constexpr int CPB = SB / LPC;             // channels of a block
    constexpr int NC = coef_count(K, true);
    constexpr int SPT = ((K + 2) * M + SB - 1) / SB;   // s / nu values a thread stages
    static_assert(CPB <= SB, "one staging thread per channel");
    const int groups = (a.C + CPB - 1) / CPB;
    const int b = blockIdx.x / groups, c0 = (blockIdx.x % groups) * CPB;
    const int tid = threadIdx.x, cl = tid / LPC, part = tid % LPC, c = c0 + cl;
    __shared__ __align__(16) float s_sn[(K + 2) * M];     // s, then nu_0 .. nu_K
    __shared__ float s_coef[NC * CPB];                     // [quantity][channel]
    // Load order: the small operands (s and nu of the sequence, and thread i < CPB's channel's
    // coefficients, kept raw) are issued first, then the state (the step's HBM traffic). Loads
    // complete in issue order, so forming the stage maps and filling LDS waits only for the small
    // ones while the state loads stay in flight, also across the barrier (which fences LDS only).
    // Every load below runs in every thread (indices clamped into range, results of the clamped
    // ones unused): loads under divergent branches would be waited for at the branch's end.
    const IO *write = static_cast<const IO *>(a.write);
    const IO *read = static_cast<const IO *>(a.read);
    IO sn[SPT];
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
        const int i = min(tid + j * SB, (K + 2) * M - 1);
        sn[j] = i < M ? write[(long long)b * M + i] : read[(long long)b * a.read_row + (i - M)];
    }
    const bool stager = tid < CPB && c0 + tid < a.C;
    const int ch = min(c0 + min(tid, CPB - 1), a.C - 1);    // the block's own channels only
    const IO *alpha = static_cast<const IO *>(a.alpha) + (long long)b * a.alpha_row + (long long)ch * K;
    const IO *beta = static_cast<const IO *>(a.beta) + (long long)b * a.beta_row + (long long)ch * K;
    const IO *rho = static_cast<const IO *>(a.rho) + (long long)b * a.rho_row + (long long)ch * (K + 1);
    IO araw[K], braw[K], rraw[K + 1];
#pragma unroll
    for (int k = 0; k < K; ++k) { araw[k] = alpha[k]; braw[k] = beta[k]; }
#pragma unroll
    for (int k = 0; k <= K; ++k) rraw[k] = rho[k];
    const IO xraw = static_cast<const IO *>(a.x)[(long long)b * a.x_row + ch];
    const IO graw = static_cast<const IO *>(a.gamma)[(long long)b * a.gamma_row + ch];
    // the flag's load without a branch (a dummy address without a mask), so nothing waits on it
    const uint8_t flag = *(a.valid ? a.valid + b : static_cast<const uint8_t *>(a.write));
    __builtin_amdgcn_sched_barrier(0);           // the small loads stay ahead of the state's
    float V[K][8];
    if constexpr (HAS_STATE) {
        const int cs = min(c, a.C - 1);
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const float4 *src = reinterpret_cast<const float4 *>(
                a.state_in + (((long long)b * K + k) * a.C + cs) * M + part * 8);
            const float4 lo = src[0], hi = src[1];
            V[k][0] = lo.x; V[k][1] = lo.y; V[k][2] = lo.z; V[k][3] = lo.w;
            V[k][4] = hi.x; V[k][5] = hi.y; V[k][6] = hi.z; V[k][7] = hi.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e) V[k][e] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < SPT; ++j)
        if (tid + j * SB < (K + 2) * M) s_sn[tid + j * SB] = to_float(sn[j]);
    // the maps in the waves that hold staging threads (a wave-uniform branch), every lane of them
    // (those past the block's channels on a clamped one), stored by the staging threads
    if (__builtin_amdgcn_readfirstlane(tid >> 6) * 64 < CPB) {
        const int radius_kind = radius_of(a.mode), rotation_kind = rotation_of(a.mode);
        float coef[NC];
#pragma unroll
        for (int k = 0; k < K; ++k)
            stage_coefficients(to_float(araw[k]), to_float(braw[k]), radius_kind, rotation_kind,
                               coef[k], coef[K + k]);
        coef[2 * K] = to_float(xraw);
#pragma unroll
        for (int k = 0; k <= K; ++k) coef[2 * K + 1 + k] = to_float(rraw[k]);
        coef[3 * K + 2] = silu(to_float(graw));
        if (stager) {
#pragma unroll
            for (int q = 0; q < NC; ++q) s_coef[q * CPB + tid] = coef[q];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (c >= a.C) return;                        // whole channel groups; no barrier follows
    const bool valid = a.valid ? flag != 0 : true;
    float y = 0.0f;
    if (valid) {
        float rc[K], rs[K];
#pragma unroll
        for (int k = 0; k < K; ++k) { rc[k] = s_coef[k * CPB + cl]; rs[k] = s_coef[(K + k) * CPB + cl]; }
        const float xv = s_coef[2 * K * CPB + cl];
        const float rcx = rc[K - 1] * xv;
        float sv[8], nv[K + 1][8];
#pragma unroll
        for (int q = 0; q <= K + 1; ++q) {
            const float4 *src = reinterpret_cast<const float4 *>(s_sn + q * M + part * 8);
            const float4 lo = src[0], hi = src[1];
            float *dst = q == 0 ? sv : nv[q - 1];
            dst[0] = lo.x; dst[1] = lo.y; dst[2] = lo.z; dst[3] = lo.w;
            dst[4] = hi.x; dst[5] = hi.y; dst[6] = hi.z; dst[7] = hi.w;
        }
        float acc[K + 1], sig = 0.0f;
#pragma unroll
        for (int k = 0; k <= K; ++k) acc[k] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            sig = fmaf(sv[e], nv[K][e], sig);
            acc[K] = fmaf(V[K - 1][e], nv[K][e], acc[K]);
            float U = fmaf(rcx, sv[e], -(rs[K - 1] * V[K - 1][e]));
#pragma unroll
            for (int k = K - 1; k >= 1; --k) {
                const float delayed = V[k - 1][e];
                const float up = rs[k - 1] * U, down = rs[k - 1] * delayed;
                V[k][e] = fmaf(rc[k - 1], delayed, up);
                U = fmaf(rc[k - 1], U, -down);
                acc[k] = fmaf(V[k][e], nv[k][e], acc[k]);
            }
            V[0][e] = U;
            acc[0] = fmaf(U, nv[0][e], acc[0]);
        }
        y = s_coef[(3 * K + 1) * CPB + cl] * fmaf(rc[K - 1], acc[K], rs[K - 1] * xv * sig);
#pragma unroll
        for (int k = 0; k < K; ++k) y = fmaf(s_coef[(2 * K + 1 + k) * CPB + cl], acc[k], y);
        y = s_coef[(3 * K + 2) * CPB + cl] * lane_sum<LPC>(y);
    }
    if (part == 0) static_cast<IO *>(a.out)[(long long)b * a.C + c] = from_float<IO>(y);
    if (a.state_out) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float4 *dst = reinterpret_cast<float4 *>(
                a.state_out + (((long long)b * K + k) * a.C + c) * M + part * 8);
            dst[0] = make_float4(V[k][0], V[k][1], V[k][2], V[k][3]);
            dst[1] = make_float4(V[k][4], V[k][5], V[k][6], V[k][7]);
        }
    }
}

// The chunked path (summary, combine, replay) with the stage map compiled in when MODE != 0.
template <typename IO, int K, int M, int MODE>
int launch_chunked(LatticeArgs &a, hipStream_t stream) {
    constexpr int L = lanes_for(K, M);
    constexpr int G = BLOCK / L;
    const long long groups = (a.C + G - 1) / G;
    if (a.chunks > 1) {
        // the summary: on the matrix cores for bf16 at K <= 4, M >= 32 and 16-token chunks
        bool summarised = false;
        if constexpr (std::is_same<IO, bf16_t>::value && K <= 4 && M >= 32) {
            if (a.chunk % summary_mfma::TT == 0) {
                constexpr int GM = summary_mfma::ROWS / K;
                const long long blocks = (long long)a.B * (a.chunks - 1) * ((a.C + GM - 1) / GM);
                hipLaunchKernelGGL((lattice_summary_mfma<K, M, MODE>), dim3(blocks), dim3(BLOCK), 0,
                                   stream, a);
                if (int rc = check_launch("lattice_summary_mfma")) return rc;
                summarised = true;
            }
        }
        if (!summarised) {
            const long long blocks = (long long)a.B * (a.chunks - 1) * groups;
            hipLaunchKernelGGL((lattice_summary<IO, K, M, MODE>), dim3(blocks), dim3(BLOCK), 0, stream, a);
            if (int rc = check_launch("lattice_summary")) return rc;
        }
        const long long threads = (long long)a.B * a.C * M;
        hipLaunchKernelGGL((lattice_combine<K>), dim3((threads + BLOCK - 1) / BLOCK), dim3(BLOCK),
                           0, stream, a);
        if (int rc = check_launch("lattice_combine")) return rc;
    }
    // A call cut finer than the plan (a training forward runs at the backward's 16-token chunks,
    // whose entering states the backward reads) replays at the planned length, entering each
    // replay chunk from every step-th chunk's state: the carries it reads shrink by that step
    // and each block scans more tokens.
    LatticeArgs r = a;
    const int plan = lattice_plan_chunk(a.B, a.T, a.C, K, M);
    if (a.chunks > 1 && plan > a.chunk && plan % a.chunk == 0) {
        r.chunk = plan;
        r.chunks = (a.T + plan - 1) / plan;
        r.carry_chunks = a.chunks;
        r.carry_step = plan / a.chunk;
    }
    const long long blocks = (long long)r.B * r.chunks * groups;
    hipLaunchKernelGGL((lattice_replay<IO, K, M, MODE>), dim3(blocks), dim3(BLOCK), 0, stream, r);
    return check_launch("lattice_replay");
}

// bf16 at the mixer's shapes runs summary and replay kernels built for their one stage map: the
// fifteen maps and the branches between them in one kernel cost 9-30 % (replay at K = 2, d_m = 64
// and 16) and 10 % (matrix-core summary) against kernels that carry one map.
__host__ __device__ constexpr bool fixed_stage_map(int K, int M) {
    return (K == 1 || K == 2 || K == 4) && (M == 16 || M == 32 || M == 64 || M == 128);
}

template <typename IO, int K, int M>
int launch_typed(LatticeArgs &a, hipStream_t stream) {
    if constexpr (step_kernel_serves(K, M)) {
        const auto aligned16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
        if (a.T == 1 && a.chunks == 1 && aligned16(a.state_in) && aligned16(a.state_out)) {
            // 1,024-thread blocks where the grid still has >= 2,048 of them (B256 C2048 K2 d_m 64:
            // 94 -> 88 us); smaller grids lost with them (B64 C2048: 23 -> 25 us), so they keep 256
            constexpr int WIDE = 1024, CPB_WIDE = WIDE / (M / 8), CPB = BLOCK / (M / 8);
            const long long wide_blocks = (long long)a.B * ((a.C + CPB_WIDE - 1) / CPB_WIDE);
            if (wide_blocks >= 2048) {
                if (a.state_in)
                    hipLaunchKernelGGL((lattice_step_kernel<IO, K, M, true, WIDE>), dim3(wide_blocks),
                                       dim3(WIDE), 0, stream, a);
                else
                    hipLaunchKernelGGL((lattice_step_kernel<IO, K, M, false, WIDE>), dim3(wide_blocks),
                                       dim3(WIDE), 0, stream, a);
                return check_launch("lattice_step_kernel");
            }
            const long long blocks = (long long)a.B * ((a.C + CPB - 1) / CPB);
            if (a.state_in)
                hipLaunchKernelGGL((lattice_step_kernel<IO, K, M, true, BLOCK>), dim3(blocks), dim3(BLOCK), 0,
                                   stream, a);
            else
                hipLaunchKernelGGL((lattice_step_kernel<IO, K, M, false, BLOCK>), dim3(blocks), dim3(BLOCK), 0,
                                   stream, a);
            return check_launch("lattice_step_kernel");
        }
    }
    if constexpr (std::is_same<IO, bf16_t>::value && fixed_stage_map(K, M)) {
        switch (a.mode) {
            case 3: return launch_chunked<IO, K, M, 3>(a, stream);
            case 6: return launch_chunked<IO, K, M, 6>(a, stream);
            case 7: return launch_chunked<IO, K, M, 7>(a, stream);
            case 8: return launch_chunked<IO, K, M, 8>(a, stream);
            case 9: return launch_chunked<IO, K, M, 9>(a, stream);
            case 10: return launch_chunked<IO, K, M, 10>(a, stream);
            case 11: return launch_chunked<IO, K, M, 11>(a, stream);
            case 12: return launch_chunked<IO, K, M, 12>(a, stream);
            case 13: return launch_chunked<IO, K, M, 13>(a, stream);
            case 14: return launch_chunked<IO, K, M, 14>(a, stream);
            case 15: return launch_chunked<IO, K, M, 15>(a, stream);
            case 16: return launch_chunked<IO, K, M, 16>(a, stream);
            case 17: return launch_chunked<IO, K, M, 17>(a, stream);
            case 18: return launch_chunked<IO, K, M, 18>(a, stream);
            case 19: return launch_chunked<IO, K, M, 19>(a, stream);
        }
    }
    return launch_chunked<IO, K, M, 0>(a, stream);
}

template <typename IO, int K>
int dispatch_m(LatticeArgs &a, hipStream_t s) {
    switch (a.M) {
        case 1: return launch_typed<IO, K, 1>(a, s);
        case 2: return launch_typed<IO, K, 2>(a, s);
        case 4: return launch_typed<IO, K, 4>(a, s);
        case 8: return launch_typed<IO, K, 8>(a, s);
        case 16: return launch_typed<IO, K, 16>(a, s);
        case 32: return launch_typed<IO, K, 32>(a, s);
        case 64: return launch_typed<IO, K, 64>(a, s);
        case 128: return launch_typed<IO, K, 128>(a, s);
    }
    return fail(MIRA_DECLINE, "lattice: unsupported d_m");
}

template <typename IO>
int dispatch_k(LatticeArgs &a, hipStream_t s) {
    switch (a.K) {
        case 1: return dispatch_m<IO, 1>(a, s);
        case 2: return dispatch_m<IO, 2>(a, s);
        case 4: return dispatch_m<IO, 4>(a, s);
        case 8: return dispatch_m<IO, 8>(a, s);
    }
    return fail(MIRA_DECLINE, "lattice: unsupported order K");
}

}  // namespace

bool lattice_supported(int K, int M, int dtype) {
    const bool k_ok = K == 1 || K == 2 || K == 4 || K == 8;
    const bool m_ok = M >= 1 && M <= 128 && (M & (M - 1)) == 0;
    return k_ok && m_ok && dtype >= MIRA_F32 && dtype <= MIRA_F16;
}

int lattice_lanes(int K, int M) { return lanes_for(K, M); }

int lattice_plan_chunk(int B, int T, int C, int K, int M) {
    // Enough (b, chunk, channel-group) blocks to put ~4 on every CU (as many as are resident at
    // once), at >= 16 tokens a chunk: longer chunks cost the summary and combine less, and at
    // B4 T2048 C2048 K2 M64 chunks of 256 tokens beat 128 by 4 % (192 and 320, which leave a
    // short last chunk, lose 15 %).
    const int G = BLOCK / lanes_for(K, M);
    const long long base = (long long)B * ((C + G - 1) / G);
    const long long target = 1024;
    if (T <= 32 || base >= target) return T;
    long long chunks = std::min<long long>((target + base - 1) / base, (T + 15) / 16);
    if (chunks <= 1) return T;
    int chunk = (int)((T + chunks - 1) / chunks);
    chunk = (chunk + 15) / 16 * 16;
    // A channel on one lane at K <= 2 (the direct-form replay and the per-slot summary) runs
    // faster at 64-token chunks than at the longer ones the block target gives: at C1536 K2 d_m 16
    // 446 against 498 us (B8 T2048, 96 planned), 810 against 938 (B8 T4096, 192), 806 against
    // 1,043 (B16 T2048, 192), 869 against 997 (B1 T32768, 192).
    if (lanes_for(K, M) == 1 && K <= 2 && chunk > 64) chunk = 64;
    return std::min(chunk, T);
}

size_t lattice_workspace(int B, int T, int C, int K, int M, int chunk) {
    if (chunk <= 0 || chunk >= T) return 0;
    const long long chunks = (T + chunk - 1) / chunk;
    const long long planes = (long long)B * chunks * C;
    return (size_t)(planes * K * K + planes * K * M) * sizeof(float);
}

int lattice_launch(LatticeArgs &a, hipStream_t stream) {
    switch (a.dtype) {
        case MIRA_F32: return dispatch_k<float>(a, stream);
        case MIRA_BF16: return dispatch_k<bf16_t>(a, stream);
        case MIRA_F16: return dispatch_k<f16_t>(a, stream);
    }
    return fail(MIRA_DECLINE, "lattice: unsupported dtype");
}

}  // namespace mira
