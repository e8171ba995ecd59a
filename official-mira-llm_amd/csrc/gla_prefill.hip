// Gated linear attention (GLA) prefill on gfx950 -- the per-row recurrent form.
//
// Per (b, head) and state row v (one value channel): S[v,:]_t = exp(g_t) S[v,:]_(t-1) + v_t[v] k_t,
// o_t[v] = S[v,:]_t . q_t. Rows are independent, so a head's 128 rows are split over 4 blocks of
// 32 rows; a half-wave owns one row (32 lanes x 4 key columns) and runs the tokens in order with
// its state in registers. This is the correctness baseline of the prefill; it does the
// recurrence on the vector ALUs and is bound by the per-token dependency chain.
#include "mira_device.hpp"
#include "mira_abi_internal.hpp"

namespace mira {
namespace {

constexpr int D = 128;
constexpr int ROWS_PER_BLOCK = 32;      // 8 half-waves x 4 rows
constexpr int THREADS = 256;
constexpr int ROWS_PER_HALF = ROWS_PER_BLOCK / (THREADS / 32);

template <typename IO>
__global__ __launch_bounds__(THREADS) void gla_recurrent_kernel(GlaArgs a) {
    const int blocks_per_head = D / ROWS_PER_BLOCK;
    const int bh = blockIdx.x / blocks_per_head;
    const int b = bh / a.H, head = bh % a.H;
    const int half = threadIdx.x >> 5;
    const int k4 = threadIdx.x & 31;
    const int row0 = (blockIdx.x % blocks_per_head) * ROWS_PER_BLOCK + half * ROWS_PER_HALF;
    float4 s[ROWS_PER_HALF];
#pragma unroll
    for (int r = 0; r < ROWS_PER_HALF; ++r) {
        const long long at = ((long long)bh * D + row0 + r) * D + 4 * k4;
        s[r] = a.S0 ? *reinterpret_cast<const float4 *>(a.S0 + at) : make_float4(0, 0, 0, 0);
    }
    const IO *q = static_cast<const IO *>(a.q);
    const IO *k = static_cast<const IO *>(a.k);
    const IO *v = static_cast<const IO *>(a.v);
    IO *o = static_cast<IO *>(a.o);
    for (int t = 0; t < a.T; ++t) {
        const long long token = ((long long)b * a.T + t) * a.H + head;
        const float decay = expf(a.g[token]);
        const IO *qt = q + token * D + 4 * k4;
        const IO *kt = k + token * D + 4 * k4;
        const float q0 = load(qt), q1 = load(qt + 1), q2 = load(qt + 2), q3 = load(qt + 3);
        const float c0 = load(kt), c1 = load(kt + 1), c2 = load(kt + 2), c3 = load(kt + 3);
#pragma unroll
        for (int r = 0; r < ROWS_PER_HALF; ++r) {
            const float vr = load(v + token * D + row0 + r);
            s[r].x = fmaf(decay, s[r].x, vr * c0);
            s[r].y = fmaf(decay, s[r].y, vr * c1);
            s[r].z = fmaf(decay, s[r].z, vr * c2);
            s[r].w = fmaf(decay, s[r].w, vr * c3);
            float part = fmaf(s[r].x, q0, fmaf(s[r].y, q1, fmaf(s[r].z, q2, s[r].w * q3)));
            part = group_sum<32>(part);
            if (k4 == 0) o[token * D + row0 + r] = from_float<IO>(part);
        }
    }
    if (a.ST) {
#pragma unroll
        for (int r = 0; r < ROWS_PER_HALF; ++r)
            *reinterpret_cast<float4 *>(a.ST + ((long long)bh * D + row0 + r) * D + 4 * k4) = s[r];
    }
}

template <typename IO>
int prefill_typed(const GlaArgs &a, hipStream_t stream) {
    const long long blocks = (long long)a.B * a.H * (D / ROWS_PER_BLOCK);
    hipLaunchKernelGGL((gla_recurrent_kernel<IO>), dim3(blocks), dim3(THREADS), 0, stream, a);
    return check_launch("gla_recurrent");
}

}  // namespace

size_t gla_workspace(int, int, int, int, int) { return 0; }

int gla_chunked_launch(const GlaArgs &a, void *, size_t, hipStream_t stream) {
    if (gla_chunk_applies(a)) return gla_chunk_launch(a, stream);
    switch (a.dtype) {
        case MIRA_F32: return prefill_typed<float>(a, stream);
        case MIRA_BF16: return prefill_typed<bf16_t>(a, stream);
        case MIRA_F16: return prefill_typed<f16_t>(a, stream);
    }
    return fail(MIRA_DECLINE, "gla: unsupported dtype");
}

}  // namespace mira
