// Gated linear attention (GLA) matrix state on gfx950: the decode step.
//
// Per (b, head): S_t = exp(g_t) S_(t-1) + k_t v_t^T, o_t = S_t^T q_t, with S stored transposed,
// [B,H,d_v,d_k] float32 -- the K=1 lattice state [B*H, 1, C=d_v, M=d_k].
//
// DECODE streams the whole state once per token (read + write, 128 KiB per head at d = 128), so it
// is HBM bound. One 256-thread block per (b, head); thread t owns the 16-byte pieces
// f = t + 256 i (i < 16) of the flattened [d_v, d_k] state, so every load and store instruction of
// a wave covers 1 KiB of contiguous HBM. Row v = f / 32 of piece f is shared by the 32 lanes of a
// half-wave, which reduce o[v] = S[v,:] . q with a butterfly.
#include "mira_device.hpp"
#include "mira_abi_internal.hpp"

namespace mira {
namespace {

constexpr int D = 128;                 // d_k = d_v
constexpr int PIECES = D * D / 4;      // float4 pieces of one head's state
constexpr int STEP_THREADS = 256;
constexpr int PER_THREAD = PIECES / STEP_THREADS;

template <typename IO>
__device__ __forceinline__ float4 load4(const IO *p) {
    return make_float4(load(p), load(p + 1), load(p + 2), load(p + 3));
}

// Sum of 16 values over the 32 lanes of each half-wave, one value per half-wave lane group:
// after the butterfly, lane l (l % 32 < 16) holds the total of value index (l % 32).
__device__ __forceinline__ float half_wave_transpose_sum(float (&v)[PER_THREAD], int lane) {
    // 16 values over 32 lanes: 16 + 8 + 4 + 2 = 30 exchanges, then one final xor-16 add.
#pragma unroll
    for (int width = PER_THREAD; width > 1; width >>= 1) {
        const int half = width >> 1;
        const int mask = half;                 // exchange partner distance in lanes
        const bool upper = (lane & mask) != 0;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float send = upper ? v[i] : v[i + half];
            const float keep = upper ? v[i + half] : v[i];
            v[i] = keep + __shfl_xor(send, mask, 64);
        }
    }
    // v[0] now holds the partial of value index (lane & 15) summed over lanes sharing lane bit 4.
    return v[0] + __shfl_xor(v[0], 16, 64);
}

template <typename IO>
__global__ __launch_bounds__(STEP_THREADS) void gla_step_kernel(GlaArgs a) {
    const int bh = blockIdx.x;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int k4 = t & 31;                             // this thread's 4 key columns
    const float decay = expf(a.g[bh]);
    const IO *q = static_cast<const IO *>(a.q) + (long long)bh * D;
    const IO *k = static_cast<const IO *>(a.k) + (long long)bh * D;
    const IO *v = static_cast<const IO *>(a.v) + (long long)bh * D;
    const float4 qv = load4(q + 4 * k4);
    const float4 kv = load4(k + 4 * k4);
    float4 *S = reinterpret_cast<float4 *>(a.ST + (long long)bh * D * D);
    float4 piece[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) piece[i] = S[t + STEP_THREADS * i];
    float part[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int row = (t >> 5) + 8 * i;
        const float vr = load(v + row);
        float4 s = piece[i];
        s.x = fmaf(decay, s.x, vr * kv.x);
        s.y = fmaf(decay, s.y, vr * kv.y);
        s.z = fmaf(decay, s.z, vr * kv.z);
        s.w = fmaf(decay, s.w, vr * kv.w);
        S[t + STEP_THREADS * i] = s;
        part[i] = fmaf(s.x, qv.x, fmaf(s.y, qv.y, fmaf(s.z, qv.z, s.w * qv.w)));
    }
    // lane l of a half-wave ends with the total of part[l & 15]: rows (t >> 5) + 8 * (l & 15)
    const float total = half_wave_transpose_sum(part, lane);
    if ((lane & 31) < 16) {
        const int row = (t >> 5) + 8 * (lane & 15);
        static_cast<IO *>(a.o)[(long long)bh * D + row] = from_float<IO>(total);
    }
}

template <typename IO>
int step_typed(const GlaArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL((gla_step_kernel<IO>), dim3(a.B * a.H), dim3(STEP_THREADS), 0, stream, a);
    return check_launch("gla_step");
}

}  // namespace

int gla_step_launch(const GlaArgs &a, hipStream_t stream) {
    switch (a.dtype) {
        case MIRA_F32: return step_typed<float>(a, stream);
        case MIRA_BF16: return step_typed<bf16_t>(a, stream);
        case MIRA_F16: return step_typed<f16_t>(a, stream);
    }
    return fail(MIRA_DECLINE, "gla: unsupported dtype");
}

}  // namespace mira
