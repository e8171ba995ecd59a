// The inference lattice scan that forms its own coefficients from the control, on gfx950: the
// reference's coefficient-forming scan (kernel/cuda/mira_dspv2/fused_scan.cuh:4-59,259-516,
// launched by matrix_lattice_iir_control, kernel/cuda/mira_dspv2/mira.py:1675-1741).
//
// alpha, beta and rho of every (token, channel) are an affine function of the token's d_r-wide
// control (the mixer's coefficient_projection):
//     coefficient[b,t,row] = bf16( sum_k control[b,t,k] W[row,k] + bias[row] )
// rounded once to bf16, as the projection's bf16 output is. Instead of reading 3K + 1 coefficients
// per (token, channel) from HBM, written there by a GEMM, the scan reads d_r control values per
// token and forms the coefficients on the matrix cores. Only the order of the d_r-term sum differs
// from the GEMM's, so a coefficient can land one bf16 ulp away.
//
// A block is SB = 16 sequences x G = 16 channels = 256 threads; each (sequence, channel) stream
// keeps its whole K x M state in the registers of one thread (K M <= 32), and the block walks the
// whole sequence (served when one token chunk covers it: the batch alone fills the GPU). The G
// channels' weight rows (alpha, beta, rho, padded to COLS rows per channel) and biases are copied
// to LDS once (d_r + 8 halfwords a row, dynamic LDS). A tile is one token of the 16 sequences:
// 16 rows, one 16-row MFMA tile, and tile n runs
//   form   control . W^T on v_mfma_f32_16x16x16_bf16 (float32 accumulation), bias added, rounded
//          to bf16, into LDS as [row][channel][column];                       barrier
//   scan   every stream forms its stage maps (r cos, r sin), rho, x and SiLU gate in registers
//          and steps (the replay's update and readout); then the inputs of tile n + 1 (control
//          rows, s and nu rows, x, gamma, valid flags) go from registers into the other half of
//          the double-buffered staging area;                                   barrier
// and the outputs of tile n leave at the start of tile n + 1. Global loads run two tiles ahead
// into two register sets that alternate by tile parity, so a tile never waits for HBM. One kernel
// per stage map (as the reference builds its fused scans): 7-14 % faster than one kernel that
// reads the map at run time. About 35 KB of LDS and at most 168 VGPRs a block: three waves per
// SIMD. The 16-sequence tile measured 20 %
// faster than 8 sequences x 2 tokens (2 blocks per CU), and forcing four waves per SIMD spilled
// and ran 29 % slower.
#include "lattice_common.hpp"
#include "mira_abi_internal.hpp"

namespace mira {
namespace {

constexpr int THREADS = 256;
constexpr int ROWS = 16;           // (sequence, token) rows of a tile: one 16-row MFMA tile
constexpr int RMAX = 64;           // widest control served
constexpr int CS = RMAX + 8;       // LDS row of a control row, halfwords (16-byte rows)

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// The (K, d_m) served: one lane holds a whole stream (K d_m <= 32) and the scan's work per
// (token, channel) is small next to the 3K + 1 coefficients it saves reading. Measured against
// the projection GEMM plus the replay (both built for the call's one stage map) at B256 T512
// C1536: 1.64x (1, 8), 1.07-1.16x (1, 16), 2.15x (2, 8), 1.38x (2, 16), 1.59x (4, 8); (1, 32)
// 0.92x and every shape whose stream spans several lanes stay on the materialised path.
__host__ __device__ constexpr bool control_serves(int K, int M) {
    return (K == 1 && (M == 8 || M == 16)) || (K == 2 && (M == 8 || M == 16)) || (K == 4 && M == 8);
}

template <int K, int M>
struct Shape {
    static constexpr int L = lanes_for(K, M);              // lanes per stream: 1
    static constexpr int TT = 1;                           // tokens per tile
    static constexpr int SB = ROWS / TT;                   // sequences per block
    static constexpr int G = 16 * TT / L;                  // channels per block
    static constexpr int MV = M / L;                       // memory slots per lane
    static constexpr int COLS = (3 * K + 1 + 7) / 8 * 8;   // weight rows per channel
    static constexpr int NCOL = G * COLS;                  // columns of the coefficient GEMM
    static constexpr int NC = coef_count(K, true);         // staged floats per (row, channel)
    // per-thread shares of a tile's loads: s and nu rows as bf16 pairs, x and gamma elements
    static constexpr int NW = (ROWS * M / 2 + THREADS - 1) / THREADS;
    static constexpr int NR = (ROWS * (K + 1) * M / 2 + THREADS - 1) / THREADS;
    static constexpr int NX = (ROWS * G + THREADS - 1) / THREADS;
    static_assert(L == 1 && SB * G * L == THREADS && NCOL % 64 == 0 && M % 2 == 0, "tile shape");
};

// Bytes of the dynamic LDS (the weight rows, stride R + 8 halfwords).
template <int K, int M>
constexpr size_t weight_bytes(int R) { return (size_t)Shape<K, M>::NCOL * (R + 8) * 2; }

__device__ __forceinline__ float bf16_value(uint32_t h) { return __uint_as_float((h & 0xffffu) << 16); }

// two floats rounded to bf16 (nearest even) in one conversion: lo in bits 0-15, hi in 16-31
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// at least three waves per SIMD: (K, d_m) = (4, 8) would otherwise take 172 VGPRs and two
template <int K, int M, int MODE>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(3)))
void lattice_control_kernel(LatticeControlArgs a) {
    using S = Shape<K, M>;
    constexpr int L = S::L, TT = S::TT, SB = S::SB, G = S::G, MV = S::MV, COLS = S::COLS;
    constexpr int NCOL = S::NCOL, NC = S::NC, NW = S::NW, NR = S::NR, NX = S::NX;
    constexpr int RW = (K + 1) * M;                        // nu floats per row
    extern __shared__ __align__(16) uint16_t s_w[];        // weight rows [NCOL][R + 8]
    __shared__ float s_bias[NCOL];
    __shared__ __align__(16) uint16_t s_ctl[2][ROWS][CS];  // control rows (double-buffered)
    __shared__ __align__(16) uint16_t s_raw[ROWS][NCOL];   // formed coefficients, bf16
    __shared__ __align__(8) float s_write[2][ROWS][M];
    __shared__ __align__(8) float s_read[2][ROWS][RW];
    __shared__ uint16_t s_xg[2][2][ROWS][G];               // raw x and gamma
    __shared__ uint16_t s_out[2][ROWS][G];
    __shared__ unsigned char s_valid[2][ROWS];

    // Workgroups go round-robin over the 8 XCDs, each with its own L2: block i runs logical block
    // (i % 8) (n / 8) + i / 8, so an XCD takes a contiguous run of channel groups of one batch
    // group -- the groups sharing a 128-byte line of x, gamma and y, and the batch group's control
    // and s rows, meet in one L2.
    const int n_blocks = gridDim.x, i_block = blockIdx.x;
    const int logical = n_blocks % 8 ? i_block : (i_block % 8) * (n_blocks / 8) + i_block / 8;
    // row r of a tile is token n TT + r / SB of sequence b0 + r % SB
    const int groups = (a.C + G - 1) / G;
    const int c0 = (logical % groups) * G, b0 = (logical / groups) * SB;
    const int tid = threadIdx.x, wave = tid >> 6, wl = tid & 63;
    const int lane = tid % L, cl = (tid / L) % G, sb = tid / (L * G);
    const int b = b0 + sb, c = c0 + cl;
    const bool active = b < a.B && c < a.C;
    const int R = a.R, WS = R + 8;
    const uint16_t *weight = static_cast<const uint16_t *>(a.weight);
    const uint16_t *bias = static_cast<const uint16_t *>(a.bias);
    const uint16_t *control = static_cast<const uint16_t *>(a.control);
    const uint16_t *xs = static_cast<const uint16_t *>(a.x);
    const uint16_t *gs = static_cast<const uint16_t *>(a.gamma);
    const uint32_t *write2 = static_cast<const uint32_t *>(a.write);
    const uint32_t *read2 = static_cast<const uint32_t *>(a.read);
    uint16_t *out = static_cast<uint16_t *>(a.out);
    const int tiles = (a.T + TT - 1) / TT;

    // ---- the block's weight rows, once: row q of a channel is alpha_q (q < K), beta_(q-K)
    // (q < 2K), rho_(q-2K) (q <= 3K), else zero padding
    auto weight_row = [&](int col) -> long long {
        const int ch = c0 + col / COLS, q = col % COLS;
        if (ch >= a.C || q > 3 * K) return -1;
        if (q < K) return a.alpha_first + (long long)ch * K + q;
        if (q < 2 * K) return a.beta_first + (long long)ch * K + (q - K);
        return a.rho_first + (long long)ch * (K + 1) + (q - 2 * K);
    };
    const int pieces = R / 4;                                  // 8-byte pieces of a weight row
    for (int i = tid; i < NCOL * pieces; i += THREADS) {
        const int col = i / pieces, piece = i % pieces;
        const long long row = weight_row(col);
        u32x2 v = {0u, 0u};
        if (row >= 0) v = *reinterpret_cast<const u32x2 *>(weight + row * a.weight_row + 4 * piece);
        *reinterpret_cast<u32x2 *>(&s_w[col * WS + 4 * piece]) = v;
    }
    for (int col = tid; col < NCOL; col += THREADS) {
        const long long row = weight_row(col);
        s_bias[col] = row >= 0 && bias ? bf16_value(bias[row]) : 0.0f;
    }

    // ---- a tile's inputs, loaded into registers two tiles ahead
    struct Pre {
        u32x4 ctl;
        uint32_t w[NW], r[NR], x[NX], g[NX];
        uint32_t valid;
    };
    const int cpieces = R / 8;                                 // 16-byte pieces of a control row
    // Every thread loads the same rows of every tile, TT tokens further on: a load slot keeps its
    // element offset at tile 0 and how many tokens its row has left (0 past the batch), so a tile
    // costs one uniform product and one add per slot instead of the whole row arithmetic.
    struct Slot { long long base; int room; };
    auto slot_of = [&](int r, long long stride, long long column) {
        const int rb = b0 + r % SB, tok = r / SB;
        return Slot{((long long)rb * a.T + tok) * stride + column, rb < a.B ? a.T - tok : 0};
    };
    const Slot none{0, 0};
    const Slot s_ctl_slot = tid < ROWS * cpieces ? slot_of(tid / cpieces, R, 8 * (tid % cpieces)) : none;
    Slot s_w_slot[NW], s_r_slot[NR], s_x_slot[NX];
    long long g_base[NX], o_base[NX];
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        const int i = tid + j * THREADS;
        s_w_slot[j] = i < ROWS * M / 2 ? slot_of(i / (M / 2), M / 2, i % (M / 2)) : none;
    }
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        const int i = tid + j * THREADS;
        s_r_slot[j] = i < ROWS * RW / 2 ? slot_of(i / (RW / 2), a.read_row / 2, i % (RW / 2)) : none;
    }
#pragma unroll
    for (int j = 0; j < NX; ++j) {
        const int i = tid + j * THREADS, r = i / G, ch = i % G;
        const bool on = i < ROWS * G && c0 + ch < a.C;
        s_x_slot[j] = on ? slot_of(r, a.x_row, c0 + ch) : none;
        g_base[j] = slot_of(r, a.gamma_row, c0 + ch).base;
        o_base[j] = slot_of(r, a.C, c0 + ch).base;
    }
    const Slot s_v_slot = tid < ROWS ? slot_of(tid, 1, 0) : none;
    auto fetch = [&](Pre &p, int n) {
        const int t0 = n * TT;
        p.ctl = u32x4{0u, 0u, 0u, 0u};
        if (t0 < s_ctl_slot.room)
            p.ctl = *reinterpret_cast<const u32x4 *>(control + s_ctl_slot.base + (long long)t0 * R);
#pragma unroll
        for (int j = 0; j < NW; ++j)
            p.w[j] = t0 < s_w_slot[j].room ? write2[s_w_slot[j].base + (long long)t0 * (M / 2)] : 0u;
#pragma unroll
        for (int j = 0; j < NR; ++j)
            p.r[j] = t0 < s_r_slot[j].room
                         ? read2[s_r_slot[j].base + (long long)t0 * (a.read_row / 2)] : 0u;
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            const bool on = t0 < s_x_slot[j].room;
            p.x[j] = on ? xs[s_x_slot[j].base + (long long)t0 * a.x_row] : 0u;
            p.g[j] = on ? gs[g_base[j] + (long long)t0 * a.gamma_row] : 0u;
        }
        p.valid = t0 < s_v_slot.room ? (!a.valid || a.valid[s_v_slot.base + t0]) : 0u;
    };
    auto stage = [&](const Pre &p, int buf) {
        if (tid < ROWS * cpieces)
            *reinterpret_cast<u32x4 *>(&s_ctl[buf][tid / cpieces][8 * (tid % cpieces)]) = p.ctl;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const int i = tid + j * THREADS, r = i / (M / 2), e = i % (M / 2);
            if (i < ROWS * M / 2)
                *reinterpret_cast<float2 *>(&s_write[buf][r][2 * e]) =
                    make_float2(bf16_value(p.w[j]), bf16_value(p.w[j] >> 16));
        }
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int i = tid + j * THREADS, r = i / (RW / 2), e = i % (RW / 2);
            if (i < ROWS * RW / 2)
                *reinterpret_cast<float2 *>(&s_read[buf][r][2 * e]) =
                    make_float2(bf16_value(p.r[j]), bf16_value(p.r[j] >> 16));
        }
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            const int i = tid + j * THREADS, r = i / G, ch = i % G;
            if (i < ROWS * G) {
                s_xg[buf][0][r][ch] = (uint16_t)p.x[j];
                s_xg[buf][1][r][ch] = (uint16_t)p.g[j];
            }
        }
        if (tid < ROWS) s_valid[buf][tid] = (unsigned char)p.valid;
    };
    auto store = [&](int n) {
        const int buf = n & 1, t0 = n * TT;
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            const int i = tid + j * THREADS;
            if (t0 < s_x_slot[j].room)
                out[o_base[j] + (long long)t0 * a.C] = s_out[buf][i / G][i % G];
        }
    };

    float V[K][MV];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int v = 0; v < MV; ++v)
            V[k][v] = active && a.state_in
                          ? a.state_in[(((long long)b * K + k) * a.C + c) * M + slot<M, L>(lane, v)]
                          : 0.0f;
    const int mode = MODE ? MODE : a.mode;             // MODE: the stage map compiled in
    const int radius_kind = radius_of(mode), rotation_kind = rotation_of(mode);

    // tile n: store n - 1, form, scan n, stage n + 1 from `use`, load n + 2 into `fill`
    auto iteration = [&](int n, Pre &fill, const Pre &use) {
        const int buf = n & 1;
        if (n + 2 < tiles) fetch(fill, n + 2);
        if (n > 0) store(n - 1);
        // ---- form: lane l gives control[l % 16][k + 4 (l / 16) ..] and W[col l % 16][same k];
        // accumulator element e of lane l is row 4 (l / 16) + e, column l % 16
        for (int ct = wave; ct < NCOL / 16; ct += 4) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            const uint16_t *wrow = &s_w[(16 * ct + (wl & 15)) * WS + 4 * (wl >> 4)];
            const uint16_t *crow = &s_ctl[buf][wl & 15][4 * (wl >> 4)];
            for (int k0 = 0; k0 < R; k0 += 16)
                acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                    *reinterpret_cast<const s16x4 *>(crow + k0),
                    *reinterpret_cast<const s16x4 *>(wrow + k0), acc, 0, 0, 0);
            const int col = 16 * ct + (wl & 15);
            const float bcol = s_bias[col];
            const uint32_t p01 = bf16_pair(acc[0] + bcol, acc[1] + bcol);
            const uint32_t p23 = bf16_pair(acc[2] + bcol, acc[3] + bcol);
            const int row = 4 * (wl >> 4);
            s_raw[row][col] = (uint16_t)p01;
            s_raw[row + 1][col] = (uint16_t)(p01 >> 16);
            s_raw[row + 2][col] = (uint16_t)p23;
            s_raw[row + 3][col] = (uint16_t)(p23 >> 16);
        }
        __syncthreads();
        // ---- scan: every stream forms its own coefficients from the raw columns, then steps;
        // a masked (or absent) row keeps the state and writes 0
        if (active) {
            float mine[TT][NC];
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                const int r = j * SB + sb;
                u32x4 raw[COLS / 8];                       // the channel's columns, 8 a piece
#pragma unroll
                for (int q = 0; q < COLS / 8; ++q)
                    raw[q] = *reinterpret_cast<const u32x4 *>(&s_raw[r][cl * COLS + 8 * q]);
                auto column = [&](int q) { return bf16_value(raw[q / 8][(q % 8) / 2] >> (16 * (q % 2))); };
#pragma unroll
                for (int k = 0; k < K; ++k)
                    stage_coefficients(column(k), column(K + k), radius_kind, rotation_kind,
                                       mine[j][k], mine[j][K + k]);
                mine[j][2 * K] = bf16_value(s_xg[buf][0][r][cl]);
#pragma unroll
                for (int k = 0; k <= K; ++k) mine[j][2 * K + 1 + k] = column(2 * K + k);
                mine[j][3 * K + 2] = silu(bf16_value(s_xg[buf][1][r][cl]));
            }
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                const int r = tt * SB + sb;
                float y = 0.0f;
                if (s_valid[buf][r])
                    y = lattice_token<K, M, L>(V, [&](int q) { return mine[tt][q]; },
                                               s_write[buf][r], s_read[buf][r], lane);
                s_out[buf][r][cl] = (uint16_t)bf16_pair(y, 0.0f);
            }
        }
        if (n + 1 < tiles) stage(use, buf ^ 1);
        __syncthreads();
    };

    Pre p0, p1;
    fetch(p0, 0);
    if (tiles > 1) fetch(p1, 1);
    stage(p0, 0);
    __syncthreads();
    for (int n = 0; n < tiles; n += 2) {
        iteration(n, p0, p1);
        if (n + 1 < tiles) iteration(n + 1, p1, p0);
    }
    store(tiles - 1);
    if (active && a.state_out) {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int v = 0; v < MV; ++v)
                a.state_out[(((long long)b * K + k) * a.C + c) * M + slot<M, L>(lane, v)] = V[k][v];
    }
}

template <int K, int M, int MODE>
int launch_km(const LatticeControlArgs &a, hipStream_t stream) {
    using S = Shape<K, M>;
    const size_t dynamic = weight_bytes<K, M>(a.R);
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(&lattice_control_kernel<K, M, MODE>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)dynamic) != hipSuccess)
        return fail(MIRA_ERR_HIP, "lattice_control_kernel: cannot raise the dynamic LDS limit");
    const long long blocks = (long long)((a.B + S::SB - 1) / S::SB) * ((a.C + S::G - 1) / S::G);
    hipLaunchKernelGGL((lattice_control_kernel<K, M, MODE>), dim3(blocks), dim3(THREADS), dynamic,
                       stream, a);
    return check_launch("lattice_control_kernel");
}

// one kernel per stage map
template <int K, int M>
int launch_mode(const LatticeControlArgs &a, hipStream_t stream) {
    switch (a.mode) {
        case 3: return launch_km<K, M, 3>(a, stream);
        case 6: return launch_km<K, M, 6>(a, stream);
        case 7: return launch_km<K, M, 7>(a, stream);
        case 8: return launch_km<K, M, 8>(a, stream);
        case 9: return launch_km<K, M, 9>(a, stream);
        case 10: return launch_km<K, M, 10>(a, stream);
        case 11: return launch_km<K, M, 11>(a, stream);
        case 12: return launch_km<K, M, 12>(a, stream);
        case 13: return launch_km<K, M, 13>(a, stream);
        case 14: return launch_km<K, M, 14>(a, stream);
        case 15: return launch_km<K, M, 15>(a, stream);
        case 16: return launch_km<K, M, 16>(a, stream);
        case 17: return launch_km<K, M, 17>(a, stream);
        case 18: return launch_km<K, M, 18>(a, stream);
        case 19: return launch_km<K, M, 19>(a, stream);
    }
    return launch_km<K, M, 0>(a, stream);
}

}  // namespace

bool lattice_control_serves(int B, int T, int C, int K, int M, int R, int dtype) {
    const bool shape = control_serves(K, M) && R >= 16 && R <= RMAX && R % 16 == 0 &&
                       dtype == MIRA_BF16;
    // one token chunk: the (sequence, channel group) blocks alone fill the GPU
    return shape && B > 0 && T > 0 && C > 0 && lattice_plan_chunk(B, T, C, K, M) >= T;
}

int lattice_control_launch(const LatticeControlArgs &a, hipStream_t stream) {
    if (a.K == 1 && a.M == 8) return launch_mode<1, 8>(a, stream);
    if (a.K == 1 && a.M == 16) return launch_mode<1, 16>(a, stream);
    if (a.K == 2 && a.M == 8) return launch_mode<2, 8>(a, stream);
    if (a.K == 2 && a.M == 16) return launch_mode<2, 16>(a, stream);
    if (a.K == 4 && a.M == 8) return launch_mode<4, 8>(a, stream);
    return fail(MIRA_DECLINE, "lattice control: unsupported (K, d_m)");
}

}  // namespace mira
