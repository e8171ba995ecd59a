// Gated linear attention (GLA) matrix state on gfx950: the decode step.
//
// Per (b, head): S_t = exp(g_t) S_(t-1) + k_t v_t^T, o_t = S_t^T q_t, with S stored transposed,
// [B,H,d_v,d_k] float32 -- the K=1 lattice state [B*H, 1, C=d_v, M=d_k].
//
// DECODE streams the whole state once per token (read + write, 128 KiB per head at d = 128), so it
// is HBM bound. One 1,024-thread block per (b, head); thread t owns the 16-byte pieces
// f = t + 1024 i (i < 4) of the flattened [d_v, d_k] state, so every load and store instruction of
// a wave covers 1 KiB of contiguous HBM. Row v = f / 32 of piece f is shared by the 32 lanes of a
// half-wave, which reduce o[v] = S[v,:] . q with a butterfly. The thread's v entries are loaded
// before the state, so the update waits on one round trip, not two.
#include "mira_device.hpp"
#include "mira_abi_internal.hpp"


namespace mira {
namespace {

constexpr int D = 128;                 // d_k = d_v
constexpr int PIECES = D * D / 4;      // float4 pieces of one head's state
// threads per (b, head): 1,024 (4 pieces each) streams the batch-256 state at 6.8 TB/s where
// 256 threads (16 pieces each) reached 6.1 and 512 threads 6.5 on the same MI355X
constexpr int STEP_THREADS = 1024;

template <typename IO>
__device__ __forceinline__ float4 load4(const IO *p) {
    return make_float4(load(p), load(p + 1), load(p + 2), load(p + 3));
}

// Sum of N values over the 32 lanes of each half-wave, one value per half-wave lane group:
// after the butterfly, lane l (l % 32 < N) holds the total of value index (l % 32).
template <int N>
__device__ __forceinline__ float half_wave_transpose_sum(float (&v)[N], int lane) {
#pragma unroll
    for (int width = N; width > 1; width >>= 1) {
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
    // v[0] now holds the partial of value index (lane % N) summed over the lanes that differ in
    // the bits above log2(N) within the half-wave
#pragma unroll
    for (int mask = N; mask < 32; mask <<= 1) v[0] += __shfl_xor(v[0], mask, 64);
    return v[0];
}

template <typename IO, int THREADS>
__global__ __launch_bounds__(THREADS) void gla_step_kernel(GlaArgs a) {
    constexpr int PER_THREAD = PIECES / THREADS;
    constexpr int ROWS = THREADS / 32;                 // state rows a pass of the block covers
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
    float vr[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) vr[i] = load(v + (t >> 5) + ROWS * i);
    float4 *S = reinterpret_cast<float4 *>(a.ST + (long long)bh * D * D);
    float4 piece[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) piece[i] = S[t + THREADS * i];
    float part[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        float4 s = piece[i];
        s.x = fmaf(decay, s.x, vr[i] * kv.x);
        s.y = fmaf(decay, s.y, vr[i] * kv.y);
        s.z = fmaf(decay, s.z, vr[i] * kv.z);
        s.w = fmaf(decay, s.w, vr[i] * kv.w);
        S[t + THREADS * i] = s;
        part[i] = fmaf(s.x, qv.x, fmaf(s.y, qv.y, fmaf(s.z, qv.z, s.w * qv.w)));
    }
    // lane l of a half-wave (l % 32 < PER_THREAD) ends with the total of part[l % 32]:
    // row (t >> 5) + ROWS (l % 32)
    const float total = half_wave_transpose_sum<PER_THREAD>(part, lane);
    if ((lane & 31) < PER_THREAD) {
        const int row = (t >> 5) + ROWS * (lane & 31);
        static_cast<IO *>(a.o)[(long long)bh * D + row] = from_float<IO>(total);
    }
}

template <typename IO>
int step_typed(const GlaArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL((gla_step_kernel<IO, STEP_THREADS>), dim3(a.B * a.H), dim3(STEP_THREADS), 0,
                       stream, a);
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
