// Gated linear attention (GLA) prefill on gfx950 matrix cores: the chunked form.
//
// Per (b, head), with the state stored transposed, S[v][k] (the lattice layout [B*H, 1, d_v, d_k]):
//     S_t = exp(g_t) S_(t-1) + v_t k_t^T,     o_t = S_t q_t
// A chunk of L = 64 tokens with in-chunk cumulative log-decay G_t = g_1 + .. + g_t gives
//     O^T   = V^T P^T + (S_in Q^T) diag(e^G)       P^T[s][t] = (k_s . q_t) e^(G_t - G_s), s <= t
//     S_out = e^(G_L) S_in + (V .* e^(G_L - G))^T K
// and every product runs on the matrix cores with float32 accumulation.
//
// One workgroup (8 waves) owns one (b, head, block of 32 value columns) and walks the chunks in
// order; the 4 blocks of a head sit on one XCD, so their shared q and k reads meet in its L2.
// Each chunk's q, k and V (raw, and decayed as a bf16 pair) are staged in LDS token-major, by all
// waves from whole-row HBM loads with 16-byte LDS writes; operands whose contraction runs over
// tokens (K^T, V^T) are read with the transposing LDS load of gfx950. Roles per chunk:
//   waves 0-2  one 32x32 tile each of the masked scores P^T (tiles (s,t) = (0,0), (1,1), (0,1);
//              the (1,0) tile is all masked) on v_mfma_f32_32x32x16_bf16, then V^T P^T for that
//              tile with the scores still in registers: an accumulator's 4-row groups are exactly
//              the B operand of v_mfma_f32_32x32x8_bf16, so P never goes through LDS.
//   wave 3     the carried-in term S_in Q^T e^G of both token halves, S_in read from a bf16 copy.
//   waves 4-7  the state: wave 4+i keeps S^T rows [32i, 32i+32) (its key block) x 32 value columns
//              as one float32 accumulator for the whole sequence and writes the bf16 copy of S.
// Partial output tiles meet in LDS: wave 0 adds the carried-in tile of tokens 0-31 to its own,
// wave 1 the carried-in tile of tokens 32-63 and wave 2's tile, and both store the chunk's
// outputs as whole 64-byte row pieces while the next chunk is computed. LDS buffers
// that cross the one barrier per chunk are double buffered by chunk parity (the decay table G,
// written two chunks ahead, is triple buffered). Global loads run two chunks ahead as raw buffer loads whose
// out-of-range offsets return zeros past the last token; stores past it are dropped the same way.
//
// Precision: the state recurrence is float32; the decayed values v e^(G_L - G_s) enter the
// state update as a bf16 high part plus its bf16 rounding remainder (~2^-16 relative), so the
// carried state loses nothing to bf16 operands beyond the bf16 inputs. The output operands (the
// decayed scores and the bf16 copy of S_in) are rounded once to bf16: ~2^-9 relative per term.
#include "mira_device.hpp"
#include "mira_abi_internal.hpp"

namespace mira {
namespace {

constexpr int L = 64;              // tokens per chunk
constexpr int DK = 128, DV = 128;  // head dims
constexpr int VB = 32;             // value columns per workgroup
constexpr int BLOCKS = DV / VB;    // workgroups per head
constexpr int THREADS = 512;       // 8 waves
// LDS row (halfwords) of a value tile, unpadded: its only reads are the transposing loads, whose
// 16-lane groups then cover the 64 banks once (a row of 16 dwords: 4 rows x 4 lanes x 2 dwords,
// the group's second half 8 dwords on); a padded row (20 dwords) put 2 lanes on a bank
constexpr int VS = VB;
constexpr int QS = DK + 8;         // LDS row (halfwords) of a feature-contiguous tile
constexpr int OS = VB + 8;         // LDS row (halfwords) of the output staging tile
constexpr unsigned OUT_OF_RANGE = 0x80000000u;
constexpr float LOG2E = 1.4426950408889634f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

struct alignas(16) Shared {
    uint16_t q[2][L][QS];          // Q of the chunk, [token][k]
    uint16_t k[2][L][QS];          // K of the chunk, [token][k]
    uint16_t vt[2][L][VS];         // V of the chunk, [token][v]
    uint16_t vh[2][L][VS];         // V e^(G_L - G_s), bf16 high part
    uint16_t vl[2][L][VS];         // its bf16 rounding remainder
    uint16_t s[2][VB][QS];         // bf16 copy of the state entering the chunk, [v][k]
    f32x4 part[2][3][4][64];       // partial output tiles: accumulator elements 4 g..4 g+3 of each lane
    uint16_t out[2][32][OS];       // waves 0, 1: a finished output tile, [token][v]
    float G[3][L];                 // in-chunk cumulative log-decay
};

// Transposed operand reads (ds_read_b64_tr_b16). Within each 16-lane group every lane gives the
// address of 4 consecutive halfwords, and lane i receives, as element j, halfword i % 4 of the
// row given by lane 4 j + i / 4 of its group. So when lane p addresses
//     row r0 + 4 (p / 32) + (p % 16) / 4,  column c0 + 16 ((p / 16) % 2) + 4 (p % 4)
// of a row-major tile, lane l receives tile[r0 + 4 (l / 32) + j][c0 + l % 32], j = 0..3: the
// 4 tokens of an MFMA operand whose contraction runs down the tile's rows.
__device__ __forceinline__ bf16x8 join(s16x4 a, s16x4 b) {
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}
__device__ __forceinline__ s16x4 read_down(const uint16_t *tile_row0_col0, int stride, int lane) {
    const uint16_t *p = tile_row0_col0 + (4 * (lane >> 5) + ((lane & 15) >> 2)) * stride +
                        16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(p));
}

// accumulator element i of a 32x32 MFMA tile sits at row drow(lane, i), column lane % 32
__device__ __forceinline__ int drow(int lane, int i) {
    return 8 * (i >> 2) + ((lane >> 5) << 2) + (i & 3);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t resource(const void *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ bf16x8 as_operand(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }

__device__ __forceinline__ bf16x8 lds_operand8(const uint16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ uint16_t to_bf16(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}

__device__ __forceinline__ float from_bf16(uint32_t h) { return __uint_as_float(h << 16); }

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                 CTRL, ROWS, 0xf, false));
}

// inclusive prefix sum over the 64 lanes: within rows of 16 by row shifts, then across rows by
// the row broadcasts of lanes 15 and 31
__device__ __forceinline__ float wave_prefix_sum(float x) {
    x += dpp<0x111, 0xf>(x);
    x += dpp<0x112, 0xf>(x);
    x += dpp<0x114, 0xf>(x);
    x += dpp<0x118, 0xf>(x);
    x += dpp<0x142, 0xa>(x);
    x += dpp<0x143, 0xc>(x);
    return x;
}

// LDS-only workgroup barrier: global loads in flight (the prefetches) and stores stay in flight
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__global__ __launch_bounds__(THREADS) void gla_chunk_kernel(GlaArgs a) {
    __shared__ Shared sh;
    // the wave index as a scalar: role branches and buffer resources stay uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;

    int bh, vb;
    if ((a.B * a.H) % 8 == 0) {                    // a head's 4 blocks on one XCD
        const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
        bh = (j >> 2) * 8 + x;
        vb = j & 3;
    } else {
        bh = blockIdx.x / BLOCKS;
        vb = blockIdx.x % BLOCKS;
    }
    const int b = bh / a.H, head = bh % a.H;
    const int chunks = (a.T + L - 1) / L;
    const unsigned row = (unsigned)a.H * DK * 2;                  // bytes between tokens
    const unsigned seq = (unsigned)a.T * row;                     // bytes of one sequence
    const long long first = ((long long)b * a.T * a.H + head) * DK;
    const __amdgpu_buffer_rsrc_t qr = resource(static_cast<const uint16_t *>(a.q) + first, seq);
    const __amdgpu_buffer_rsrc_t kr = resource(static_cast<const uint16_t *>(a.k) + first, seq);
    const __amdgpu_buffer_rsrc_t vr =
        resource(static_cast<const uint16_t *>(a.v) + first + vb * VB, seq);
    const __amdgpu_buffer_rsrc_t orr = resource(static_cast<uint16_t *>(a.o) + first + vb * VB, seq);
    const __amdgpu_buffer_rsrc_t gr =
        resource(a.g + (long long)b * a.T * a.H + head, (unsigned)a.T * a.H * 4);
    auto token_offset = [&](int t, unsigned within) {
        return t < a.T ? (unsigned)t * row + within : OUT_OF_RANGE;
    };

    // ---- staging, two chunks ahead: wave w loads tokens [16 (w % 4), +16) of q (w < 4) or k
    // (w >= 4) as 4 row-quads (lane: token 4 r + lane / 16, 16-byte piece lane % 16); waves 4-7
    // also V tokens [16 (w - 4), +16) (lane: token lane / 4, piece lane % 4); wave 3, the lightest,
    // the decays of the chunk after (and their prefix sum when staging). Two register sets alternate by chunk parity.
    const bool loads_q = wave < 4;
    const int kb = wave - 4;                                          // state waves' key block
    struct Staged { u32x4 rows[4], v; float g; };
    Staged set0, set1;
    auto load_decay = [&](int chunk) {
        const int t = chunk * L + lane;
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             gr, t < a.T ? (unsigned)t * a.H * 4 : OUT_OF_RANGE, 0, 0));
    };
    auto load_chunk = [&](Staged &in, int chunk) {
        const int t0 = chunk * L + 16 * (wave & 3);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            in.rows[r] = __builtin_amdgcn_raw_buffer_load_b128(
                loads_q ? qr : kr, token_offset(t0 + 4 * r + (lane >> 4), (lane & 15) * 16), 0, 0);
        if (!loads_q)
            in.v = __builtin_amdgcn_raw_buffer_load_b128(
                vr, token_offset(t0 + (lane >> 2), (lane & 3) * 16), 0, 0);
        if (wave == 3) in.g = load_decay(chunk + 1);
    };
    float gl = 1.0f;                                                  // state waves: e^(G_L)
    // stage chunk n from registers; G_s, G_L from the decay table (or `local` in the prologue)
    auto stage = [&](int n, const Staged &in, const float *local) {
        const int buf = n & 1, row0 = 16 * (wave & 3);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint16_t *dst = loads_q ? &sh.q[buf][row0 + 4 * r + (lane >> 4)][(lane & 15) * 8]
                                    : &sh.k[buf][row0 + 4 * r + (lane >> 4)][(lane & 15) * 8];
            *reinterpret_cast<u32x4 *>(dst) = in.rows[r];
        }
        if (!loads_q) {
            const int s = row0 + (lane >> 2), v0 = 8 * (lane & 3);
            const float GL = local ? local[1] : sh.G[n % 3][L - 1];
            const float Gs = local ? local[0] : sh.G[n % 3][s];
            gl = __builtin_amdgcn_exp2f(GL * LOG2E);
            const float scale = __builtin_amdgcn_exp2f((GL - Gs) * LOG2E);
            u32x4 hi, lo;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float w0 = from_bf16(in.v[j] & 0xffffu) * scale;
                const float w1 = __uint_as_float(in.v[j] & 0xffff0000u) * scale;
                hi[j] = pack_bf16(w0, w1);
                lo[j] = pack_bf16(w0 - from_bf16(hi[j] & 0xffffu), w1 - __uint_as_float(hi[j] & 0xffff0000u));
            }
            *reinterpret_cast<u32x4 *>(&sh.vt[buf][s][v0]) = in.v;
            *reinterpret_cast<u32x4 *>(&sh.vh[buf][s][v0]) = hi;
            *reinterpret_cast<u32x4 *>(&sh.vl[buf][s][v0]) = lo;
        }
    };

    // ---- prologue: chunk 0 staged, chunk 1 loading, decay tables of chunks 0 and 1
    f32x16 S = {};                                                    // state waves
    const long long srow = ((long long)bh * DV + vb * VB + col) * DK + 32 * kb + 4 * half;
    load_chunk(set0, 0);
    load_chunk(set1, 1);
    if (!loads_q) {
        if (a.S0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 s4 = *reinterpret_cast<const float4 *>(a.S0 + srow + 8 * j);
                S[4 * j] = s4.x; S[4 * j + 1] = s4.y; S[4 * j + 2] = s4.z; S[4 * j + 3] = s4.w;
            }
        }
        const float G0 = wave_prefix_sum(load_decay(0));
        if (kb == 0) sh.G[0][lane] = G0;
        const float local[2] = {__shfl(G0, 16 * kb + (lane >> 2), 64),
                                __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                              __builtin_bit_cast(int, G0), 63))};
        stage(0, set0, local);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<u32x2 *>(&sh.s[0][col][32 * kb + 8 * j + 4 * half]) =
                u32x2{pack_bf16(S[4 * j], S[4 * j + 1]), pack_bf16(S[4 * j + 2], S[4 * j + 3])};
    } else {
        stage(0, set0, nullptr);
        if (wave == 3) sh.G[1][lane] = wave_prefix_sum(set0.g);
    }
    lds_barrier();

    auto put_part = [&](f32x4 (&dst)[4][64], const f32x16 &v) {
#pragma unroll
        for (int g = 0; g < 4; ++g) dst[g][lane] = f32x4{v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
    };
    auto add_part = [&](f32x16 &v, const f32x4 (&src)[4][64]) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 x = src[g][lane];
            v[4 * g] += x[0]; v[4 * g + 1] += x[1]; v[4 * g + 2] += x[2]; v[4 * g + 3] += x[3];
        }
    };
    f32x16 kept = {};                                                 // waves 0, 1: last tile
    // waves 0, 1: add the partial tiles of chunk `chunk`, store its 32 tokens x 32 values
    auto finish = [&](int chunk) {
        const int buf = chunk & 1;
        f32x16 total = kept;
        add_part(total, sh.part[buf][wave == 0 ? 1 : 2]);
        if (wave == 1) add_part(total, sh.part[buf][0]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<u32x2 *>(&sh.out[wave][col][8 * j + 4 * half]) =
                u32x2{pack_bf16(total[4 * j], total[4 * j + 1]),
                      pack_bf16(total[4 * j + 2], total[4 * j + 3])};
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int r = 16 * m + (lane >> 2);
            const u32x4 piece = *reinterpret_cast<const u32x4 *>(&sh.out[wave][r][8 * (lane & 3)]);
            __builtin_amdgcn_raw_buffer_store_b128(
                piece, orr, token_offset(chunk * L + 32 * wave + r, (lane & 3) * 16), 0, 0);
        }
    };

    // iteration c: load chunk c + 2 into `fill`, compute chunk c, stage chunk c + 1 from `use`
    auto iteration = [&](int c, Staged &fill, const Staged &use) {
        const int buf = c & 1;
        const float *G = sh.G[c % 3];
        load_chunk(fill, c + 2);
        if (wave < 3) {
            if (wave < 2 && c > 0) finish(c - 1);
            const int sb = wave == 1 ? 1 : 0, tb = wave == 0 ? 0 : 1;
            // two accumulation chains (even and odd key steps), added at the end
            f32x16 acc = {}, acc2 = {};
#pragma unroll
            for (int kk = 0; kk < 8; kk += 2) {
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    lds_operand8(&sh.k[buf][32 * sb + col][16 * kk + 8 * half]),
                    lds_operand8(&sh.q[buf][32 * tb + col][16 * kk + 8 * half]), acc, 0, 0, 0);
                acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    lds_operand8(&sh.k[buf][32 * sb + col][16 * kk + 16 + 8 * half]),
                    lds_operand8(&sh.q[buf][32 * tb + col][16 * kk + 16 + 8 * half]), acc2, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] += acc2[i];
            const int t = 32 * tb + col;
            const float Gt = G[t];
            f32x16 out = {};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int s0 = 32 * sb + 8 * j + 4 * half;
                const f32x4 Gs = *reinterpret_cast<const f32x4 *>(&G[s0]);
                float p[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float decay = __builtin_amdgcn_exp2f((Gt - Gs[e]) * LOG2E);
                    p[e] = s0 + e <= t ? acc[4 * j + e] * decay : 0.0f;
                }
                const s16x4 pb = __builtin_bit_cast(s16x4, u32x2{pack_bf16(p[0], p[1]),
                                                                 pack_bf16(p[2], p[3])});
                out = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(
                    read_down(&sh.vt[buf][32 * sb + 8 * j][0], VS, lane), pb, out, 0, 0, 0);
            }
            if (wave == 2) {
                put_part(sh.part[buf][0], out);
            } else {
                kept = out;
            }
        } else if (wave == 3) {
            // the carried-in term S_in Q^T e^G of both token halves, sharing the S_in operand
            f32x16 acc0 = {}, acc1 = {};
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const bf16x8 sop = lds_operand8(&sh.s[buf][col][16 * kk + 8 * half]);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    sop, lds_operand8(&sh.q[buf][col][16 * kk + 8 * half]), acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    sop, lds_operand8(&sh.q[buf][32 + col][16 * kk + 8 * half]), acc1, 0, 0, 0);
            }
            const float g0 = __builtin_amdgcn_exp2f(G[col] * LOG2E);
            const float g1 = __builtin_amdgcn_exp2f(G[32 + col] * LOG2E);
            put_part(sh.part[buf][1], acc0 * g0);
            put_part(sh.part[buf][2], acc1 * g1);
        } else {
            // S^T[32 kb + drow][col] = S[v = col][k = 32 kb + drow]
#pragma unroll
            for (int i = 0; i < 16; ++i) S[i] *= gl;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                // the 16 tokens of step kk as two transposed reads: element i of lane half h is
                // token 16 kk + 4 h + i (i < 4) or 16 kk + 8 + 4 h + (i - 4), the same
                // permutation of the contraction in both operands
                const int r0 = 16 * kk;
                const bf16x8 kop = join(read_down(&sh.k[buf][r0][32 * kb], QS, lane),
                                        read_down(&sh.k[buf][r0 + 8][32 * kb], QS, lane));
                const bf16x8 vho = join(read_down(&sh.vh[buf][r0][0], VS, lane),
                                        read_down(&sh.vh[buf][r0 + 8][0], VS, lane));
                const bf16x8 vlo = join(read_down(&sh.vl[buf][r0][0], VS, lane),
                                        read_down(&sh.vl[buf][r0 + 8][0], VS, lane));
                S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, vho, S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, vlo, S, 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<u32x2 *>(&sh.s[buf ^ 1][col][32 * kb + 8 * j + 4 * half]) =
                    u32x2{pack_bf16(S[4 * j], S[4 * j + 1]), pack_bf16(S[4 * j + 2], S[4 * j + 3])};
        }
        if (c + 1 < chunks) {
            stage(c + 1, use, nullptr);
            if (wave == 3) sh.G[(c + 2) % 3][lane] = wave_prefix_sum(use.g);
        }
        lds_barrier();
    };
    for (int c = 0; c < chunks; c += 2) {
        iteration(c, set0, set1);
        if (c + 1 < chunks) iteration(c + 1, set1, set0);
    }
    if (wave < 2) finish(chunks - 1);
    if (!loads_q && a.ST) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<float4 *>(a.ST + srow + 8 * j) =
                make_float4(S[4 * j], S[4 * j + 1], S[4 * j + 2], S[4 * j + 3]);
    }
}

}  // namespace

// bf16 inputs, aligned rows and per-sequence extents that fit 32-bit buffer offsets; other cases
// take the per-row recurrent kernel
bool gla_chunk_applies(const GlaArgs &a) {
    const auto aligned = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return a.dtype == MIRA_BF16 && a.dk == DK && a.dv == DV && aligned(a.q) && aligned(a.k) &&
           aligned(a.v) && aligned(a.o) &&
           (unsigned long long)a.T * a.H * DK * 2 < OUT_OF_RANGE;
}

int gla_chunk_launch(const GlaArgs &a, hipStream_t stream) {
    const long long blocks = (long long)a.B * a.H * BLOCKS;
    hipLaunchKernelGGL(gla_chunk_kernel, dim3(blocks), dim3(THREADS), 0, stream, a);
    return check_launch("gla_chunk");
}

}  // namespace mira
