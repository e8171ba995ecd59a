// Depthwise causal conv (width W) + diagonal decay scan, prefill and decode, on gfx950.
//
//     u_t = sum_j w[d,j] x_(t-W+1+j) + bias[d],     h_t = a_t h_(t-1) + (1 - a_t) u_t,     y_t = h_t
//
// PREFILL IS ONE PASS OVER HBM. The work is cut into tiles of 64 tokens x TILE_C channels; a tile
// is one wave (64 lanes = 4 token groups x 16 channel lanes, 16 tokens x VEC channels per lane,
// VEC = 4 channels = one 8-byte load in bf16). A tile's map h_in -> h_out is affine, (A, H) with
// A = prod a and H the state reached from zero, so the tiles of one (sequence, channel block) --
// a chain -- are joined by a decoupled look-back: each tile publishes its aggregate (A, H) as soon
// as its inputs are in registers, folds its predecessors' aggregates back to the nearest
// published inclusive state, publishes its own inclusive state, and only then replays its 16
// tokens per lane from registers and stores y. x and a are read once and y written once:
// 6 bytes per (b, t, d) in bf16.
//
// Forward progress: a tile index is a ticket drawn from the chain's counter by a running wave,
// so every tile a wave waits on is held by a wave that is already running (or done); the waits
// are nevertheless bounded, and a wait that runs out sets the workspace's watchdog word.
// Counters return to zero at the end of every launch; flags carry a per-launch epoch, so the
// workspace needs zero-filling only once, when it is allocated.
#include "mira_device.hpp"
#include "mira_abi_internal.hpp"

#include <atomic>

namespace mira {
namespace {

constexpr int CL = 16;            // channel lanes per wave
constexpr int TG = 4;             // token groups per wave
// tokens per lane: 16 of a 16-bit type (8-byte packs), 8 of float32 (16-byte packs), so a lane
// holds 32 registers of x and 32 of a either way
__host__ __device__ constexpr int tokens_per_lane(int element_bytes) { return element_bytes == 4 ? 8 : 16; }
constexpr unsigned SPIN_LIMIT = 1u << 22;

// Four channels per lane: one 8-byte load of a 16-bit type, one 16-byte load of float32.
constexpr int VEC = 4;
template <typename IO> struct Raw { typedef uint2 type; };
template <> struct Raw<float> { typedef uint4 type; };

template <typename IO>
__device__ __forceinline__ typename Raw<IO>::type raw_zero() {
    typename Raw<IO>::type r;
    __builtin_memset(&r, 0, sizeof(r));
    return r;
}

template <typename IO>
__device__ __forceinline__ void unpack(const typename Raw<IO>::type &p, float (&f)[VEC]) {
    if constexpr (sizeof(IO) == 4) {
        f[0] = __uint_as_float(p.x); f[1] = __uint_as_float(p.y);
        f[2] = __uint_as_float(p.z); f[3] = __uint_as_float(p.w);
    } else {
        const uint32_t words[2] = {p.x, p.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint16_t lo = words[i] & 0xffffu, hi = words[i] >> 16;
            IO l, h;
            __builtin_memcpy(&l, &lo, 2);
            __builtin_memcpy(&h, &hi, 2);
            f[2 * i] = to_float(l);
            f[2 * i + 1] = to_float(h);
        }
    }
}

template <typename IO>
__device__ __forceinline__ typename Raw<IO>::type pack(const float (&f)[VEC]) {
    typename Raw<IO>::type p;
    if constexpr (sizeof(IO) == 4) {
        p.x = __float_as_uint(f[0]); p.y = __float_as_uint(f[1]);
        p.z = __float_as_uint(f[2]); p.w = __float_as_uint(f[3]);
    } else {
        uint32_t words[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const IO l = from_float<IO>(f[2 * i]), h = from_float<IO>(f[2 * i + 1]);
            uint16_t lo, hi;
            __builtin_memcpy(&lo, &l, 2);
            __builtin_memcpy(&hi, &h, 2);
            words[i] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        p.x = words[0]; p.y = words[1];
    }
    return p;
}

template <typename IO>
__device__ __forceinline__ typename Raw<IO>::type load_raw(const IO *p) {
    return *reinterpret_cast<const typename Raw<IO>::type *>(p);
}

template <typename IO>
__device__ __forceinline__ void store_raw(IO *p, const typename Raw<IO>::type &v) {
    *reinterpret_cast<typename Raw<IO>::type *>(p) = v;
}

// PUBLICATION WITHOUT AN L2 WRITE-BACK. A release fence at agent scope writes back the whole L2
// of the issuing XCD, and a tile publishes twice, so the published records are instead written
// and read with agent-scope relaxed atomics, which go to the device coherence point instead of
// the XCD's non-coherent L2; the writer waits for its record stores to complete (vmcnt(0))
// before it stores the flag, and a reader loads a record only after it has seen the flag.
__device__ __forceinline__ void publish_value(float *p, float v) {
    __hip_atomic_store(reinterpret_cast<unsigned *>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_pair(float2 *p, float a, float h) {
    const unsigned long long bits =
        (unsigned long long)__float_as_uint(a) | ((unsigned long long)__float_as_uint(h) << 32);
    __hip_atomic_store(reinterpret_cast<unsigned long long *>(p), bits, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float read_value(const float *p) {
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<const unsigned *>(p),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ float2 read_pair(const float2 *p) {
    const unsigned long long bits = __hip_atomic_load(
        reinterpret_cast<const unsigned long long *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((unsigned)bits), __uint_as_float((unsigned)(bits >> 32)));
}
// every store this wave has issued has completed at its coherence point
__device__ __forceinline__ void stores_complete() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void set_flag(unsigned *flag, unsigned value) {
    __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workspace layout (bytes): [0,256) watchdog word | counters[chains] | flags[chains*tiles]
// | aggregates (A,H)[chains*tiles*TILE_C] | inclusive H[chains*tiles*TILE_C]
struct Layout {
    long long chains, tiles, tile_c;
    size_t counters, flags, agg, inc, total;
};

__host__ __device__ inline Layout layout(int B, int T, int D, int vec, int element_bytes) {
    const int TILE_T = TG * tokens_per_lane(element_bytes);
    Layout l;
    l.tile_c = (long long)CL * vec;
    l.chains = (long long)B * ((D + l.tile_c - 1) / l.tile_c);
    l.tiles = (T + TILE_T - 1) / TILE_T;
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    l.counters = 256;
    l.flags = l.counters + up(l.chains * 4);
    l.agg = l.flags + up(l.chains * l.tiles * 4);
    l.inc = l.agg + up(l.chains * l.tiles * l.tile_c * 8);
    l.total = l.inc + up(l.chains * l.tiles * l.tile_c * 4);
    return l;
}

template <typename IO, int W>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3))) void diag_scan_kernel(DiagArgs a, unsigned char *ws,
                                                       unsigned epoch) {
    constexpr int TILE_C = CL * VEC;
    constexpr int H = W - 1;                         // conv history
    typedef typename Raw<IO>::type RawT;
    constexpr int TPT = tokens_per_lane(sizeof(IO));
    constexpr int TILE_T = TG * TPT;
    const Layout lay = layout(a.B, a.T, a.D, VEC, sizeof(IO));
    unsigned *watchdog = reinterpret_cast<unsigned *>(ws);
    unsigned *counters = reinterpret_cast<unsigned *>(ws + lay.counters);
    unsigned *flags = reinterpret_cast<unsigned *>(ws + lay.flags);
    float2 *agg = reinterpret_cast<float2 *>(ws + lay.agg);
    float *inc = reinterpret_cast<float *>(ws + lay.inc);

    const int lane = threadIdx.x;
    const int tg = lane >> 4, cl = lane & 15;
    const int chain = blockIdx.x % lay.chains;
    unsigned ticket = 0;
    if (lane == 0) {
        ticket = atomicAdd(counters + chain, 1u);
        if (ticket == lay.tiles - 1)                 // every ticket of this chain is drawn
            __hip_atomic_store(counters + chain, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int tile = __shfl(ticket, 0);
    const int cblocks = (a.D + TILE_C - 1) / TILE_C;
    const int b = chain / cblocks;
    const int d0 = (chain % cblocks) * TILE_C + cl * VEC;
    const bool dact = d0 < a.D;
    const int t0 = tile * TILE_T + tg * TPT;
    const long long row0 = (long long)b * a.T;

    // per-channel conv weights
    float wv[VEC][W], bias[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
#pragma unroll
        for (int j = 0; j < W; ++j) wv[e][j] = dact ? a.w[(long long)(d0 + e) * W + j] : 0.0f;
        bias[e] = (dact && a.bias) ? a.bias[d0 + e] : 0.0f;
    }

    // this lane's 16 tokens of x and a, as raw packs
    RawT xp[TPT], ap[TPT];
    const IO *x = static_cast<const IO *>(a.x);
    const IO *av = static_cast<const IO *>(a.a);
    // a wave-uniform base per sequence and a 32-bit byte offset per lane (T * D elements of one
    // sequence fit in 4 GiB, checked by the host), so each access needs one offset register
    const char *xs = reinterpret_cast<const char *>(x + row0 * a.D);
    const char *as = reinterpret_cast<const char *>(av + row0 * a.D);
    const uint32_t lane_off = ((uint32_t)t0 * (uint32_t)a.D + (uint32_t)d0) * (uint32_t)sizeof(IO);
    const uint32_t row_bytes = (uint32_t)a.D * (uint32_t)sizeof(IO);
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
        const int t = t0 + i;
        if (dact && t < a.T) {
            xp[i] = *reinterpret_cast<const RawT *>(xs + (lane_off + i * row_bytes));
            ap[i] = *reinterpret_cast<const RawT *>(as + (lane_off + i * row_bytes));
        } else {
            xp[i] = raw_zero<IO>();
            ap[i] = raw_zero<IO>();
        }
    }

    // conv history: the H tokens before t0, from the previous token group's registers, or (first
    // group) from HBM, the ring, or zero
    float hist[H][VEC];
#pragma unroll
    for (int j = 0; j < H; ++j) {
        RawT p;
        uint32_t *pw = reinterpret_cast<uint32_t *>(&p);
        const uint32_t *sw = reinterpret_cast<const uint32_t *>(&xp[TPT - H + j]);
#pragma unroll
        for (int word = 0; word < (int)(sizeof(RawT) / 4); ++word)
            pw[word] = __shfl(sw[word], (lane - 16) & 63);
        float f[VEC];
        unpack<IO>(p, f);
        if (tg == 0) {
            const int t = t0 - H + j;                  // token index local to this call
            const long long stream = a.pos + t;        // index in the whole stream
#pragma unroll
            for (int e = 0; e < VEC; ++e) f[e] = 0.0f;
            if (dact && t >= 0) {
                unpack<IO>(load_raw(x + (row0 + t) * a.D + d0), f);
            } else if (dact && stream >= 0 && a.ring_in) {
                const IO *ring = static_cast<const IO *>(a.ring_in);
                const int s = (int)(stream % H);
#pragma unroll
                for (int e = 0; e < VEC; ++e)
                    f[e] = load(ring + ((long long)b * a.D + d0 + e) * H + s);
            }
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) hist[j][e] = f[e];
    }

    // local scan from zero: the lane's map (A, H) over its tokens
    float A[VEC], Hs[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) { A[e] = 1.0f; Hs[e] = 0.0f; }
    {
        float win[H][VEC];
#pragma unroll
        for (int j = 0; j < H; ++j)
#pragma unroll
            for (int e = 0; e < VEC; ++e) win[j][e] = hist[j][e];
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            float xf[VEC], af[VEC];
            unpack<IO>(xp[i], xf);
            unpack<IO>(ap[i], af);
            const bool live = t0 + i < a.T;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float u = bias[e];
#pragma unroll
                for (int j = 0; j < H; ++j) u = fmaf(wv[e][j], win[j][e], u);
                u = fmaf(wv[e][H], xf[e], u);
                if (live) {
                    Hs[e] = fmaf(af[e], Hs[e], (1.0f - af[e]) * u);
                    A[e] *= af[e];
                }
#pragma unroll
                for (int j = 0; j + 1 < H; ++j) win[j][e] = win[j + 1][e];
                win[H - 1][e] = xf[e];
            }
        }
    }

    // The replay below recomputes the conv and unpacks x and a again from the raw packs rather
    // than keeping 2 x 16 x VEC floats alive across the look-back: hide the packs' values from
    // the optimiser so that it cannot reuse the first pass's results.
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
        uint32_t *xw = reinterpret_cast<uint32_t *>(&xp[i]);
        uint32_t *aw = reinterpret_cast<uint32_t *>(&ap[i]);
#pragma unroll
        for (int word = 0; word < (int)(sizeof(RawT) / 4); ++word) {
            asm volatile("" : "+v"(xw[word]));
            asm volatile("" : "+v"(aw[word]));
        }
    }

    // inclusive scan of the four token groups' maps (later o earlier = (A_l A_e, A_l H_e + H_l))
#pragma unroll
    for (int offset = 16; offset < 64; offset <<= 1) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const float pa = __shfl_up(A[e], offset, 64);
            const float ph = __shfl_up(Hs[e], offset, 64);
            if (lane >= offset) {
                Hs[e] = fmaf(A[e], ph, Hs[e]);
                A[e] *= pa;
            }
        }
    }
    float Ae[VEC], He[VEC], At[VEC], Ht[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        const float pa = __shfl_up(A[e], 16, 64), ph = __shfl_up(Hs[e], 16, 64);
        Ae[e] = tg == 0 ? 1.0f : pa;                    // this group's exclusive in-tile map
        He[e] = tg == 0 ? 0.0f : ph;
        At[e] = __shfl(A[e], 48 + cl, 64);              // the whole tile's map
        Ht[e] = __shfl(Hs[e], 48 + cl, 64);
    }

    const long long slot = (long long)chain * lay.tiles + tile;
    const unsigned tag = (epoch & 0x3fffffffu) << 2;
    float hin[VEC];
    if (tile == 0) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
            hin[e] = (dact && a.h0) ? a.h0[(long long)b * a.D + d0 + e] : 0.0f;
    } else {
        // publish the aggregate
        if (tg == 3) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) publish_pair(agg + slot * TILE_C + cl * VEC + e, At[e], Ht[e]);
        }
        stores_complete();
        if (lane == 48)
            set_flag(flags + slot, tag | 1u);
        // look back: token group g inspects predecessor base - g
        float cA[VEC], cH[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) { cA[e] = 1.0f; cH[e] = 0.0f; hin[e] = 0.0f; }
        long long base = tile - 1;
        unsigned spins = 0;
        while (true) {
            const long long p = base - tg;
            unsigned status = 2;
            if (p >= 0) {
                const unsigned f = __hip_atomic_load(flags + (long long)chain * lay.tiles + p,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                status = (f & ~3u) == tag ? (f & 3u) : 0u;
            }
            const unsigned long long ready = __ballot(status >= 1 && cl == 0);
            const unsigned long long inclusive = __ballot(status == 2 && cl == 0);
            int first_inclusive = 4;
#pragma unroll
            for (int g = 3; g >= 0; --g)
                if ((inclusive >> (16 * g)) & 1ull) first_inclusive = g;
            bool all_ready = true;
            for (int g = 0; g < first_inclusive; ++g)
                if (!((ready >> (16 * g)) & 1ull)) all_ready = false;
            if (!all_ready) {
                if (++spins > SPIN_LIMIT) {
                    if (lane == 0)
                        __hip_atomic_store(watchdog, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
                continue;
            }
            float pA[VEC], pH[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) { pA[e] = 1.0f; pH[e] = 0.0f; }
            if (p >= 0 && tg < first_inclusive) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float2 v = read_pair(agg + (base - tg + (long long)chain * lay.tiles) * TILE_C + cl * VEC + e);
                    pA[e] = v.x; pH[e] = v.y;
                }
            } else if (p >= 0 && tg == first_inclusive) {
#pragma unroll
                for (int e = 0; e < VEC; ++e)
                    pH[e] = read_value(inc + (base - tg + (long long)chain * lay.tiles) * TILE_C + cl * VEC + e);
            }
            const int last = first_inclusive < 4 ? first_inclusive : 3;
            for (int g = 0; g <= last; ++g) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float ga = __shfl(pA[e], 16 * g + cl, 64);
                    const float gh = __shfl(pH[e], 16 * g + cl, 64);
                    if (g < first_inclusive) {         // fold one more aggregate: c o F_p
                        cH[e] = fmaf(cA[e], gh, cH[e]);
                        cA[e] *= ga;
                    } else {                           // the inclusive state ends the walk
                        hin[e] = fmaf(cA[e], gh, cH[e]);
                    }
                }
            }
            if (first_inclusive < 4) break;
            base -= 4;
        }
    }
    // publish this tile's inclusive state
    if (tg == 3) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) publish_value(inc + slot * TILE_C + cl * VEC + e, fmaf(At[e], hin[e], Ht[e]));
    }
    stores_complete();
    if (lane == 48) set_flag(flags + slot, tag | 2u);

    // replay the lane's tokens from its entering state and store y
    float h[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) h[e] = fmaf(Ae[e], hin[e], He[e]);
    IO *y = static_cast<IO *>(a.y);
    char *ys = reinterpret_cast<char *>(y + row0 * a.D);
    {
        float win[H][VEC];
#pragma unroll
        for (int j = 0; j < H; ++j)
#pragma unroll
            for (int e = 0; e < VEC; ++e) win[j][e] = hist[j][e];
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            float xf[VEC], af[VEC], out[VEC];
            unpack<IO>(xp[i], xf);
            unpack<IO>(ap[i], af);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float u = bias[e];
#pragma unroll
                for (int j = 0; j < H; ++j) u = fmaf(wv[e][j], win[j][e], u);
                u = fmaf(wv[e][H], xf[e], u);
                h[e] = fmaf(af[e], h[e], (1.0f - af[e]) * u);
                out[e] = h[e];
#pragma unroll
                for (int j = 0; j + 1 < H; ++j) win[j][e] = win[j + 1][e];
                win[H - 1][e] = xf[e];
            }
            const int t = t0 + i;
            if (dact && t < a.T)
                *reinterpret_cast<RawT *>(ys + (lane_off + i * row_bytes)) = pack<IO>(out);
            if (dact && t == a.T - 1 && a.hT) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) a.hT[(long long)b * a.D + d0 + e] = h[e];
            }
        }
    }

    // the ring after this call: the last H stream tokens, each in slot (stream index mod H)
    if (a.ring_out && tile == lay.tiles - 1 && tg == 0 && dact) {
        const IO *ring_in = static_cast<const IO *>(a.ring_in);
        IO *ring_out = static_cast<IO *>(a.ring_out);
#pragma unroll
        for (int j = 0; j < H; ++j) {
            const long long stream = a.pos + a.T - H + j;   // one of the last H stream tokens
            const long long t = a.T - H + j;                // its index in this call
            const int s = (int)(((stream % H) + H) % H);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const long long at = ((long long)b * a.D + d0 + e) * H + s;
                if (stream < 0) ring_out[at] = from_float<IO>(0.0f);
                else if (t >= 0) ring_out[at] = x[(row0 + t) * a.D + d0 + e];
                else if (!ring_in) ring_out[at] = from_float<IO>(0.0f);
                else if (ring_in != ring_out) ring_out[at] = ring_in[at];
            }
        }
    }
}

// one decode token: thread per VEC channels of one sequence
template <typename IO, int W>
__global__ __launch_bounds__(256) void diag_step_kernel(DiagArgs a, float *hstate) {
    constexpr int H = W - 1;
    const long long index = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long per_row = a.D / VEC;
    if (index >= (long long)a.B * per_row) return;
    const int b = index / per_row;
    const int d0 = (index % per_row) * VEC;
    const IO *x = static_cast<const IO *>(a.x);
    const IO *av = static_cast<const IO *>(a.a);
    IO *ring = static_cast<IO *>(a.ring_out);
    const long long at = (long long)b * a.D + d0;
    float xf[VEC], af[VEC], h[VEC], out[VEC];
    unpack<IO>(load_raw(x + at), xf);
    unpack<IO>(load_raw(av + at), af);
    {
        const float4 v = *reinterpret_cast<const float4 *>(hstate + at);
        h[0] = v.x; h[1] = v.y; h[2] = v.z; h[3] = v.w;
    }
    const int write_slot = (int)(a.pos % H);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        const long long d = d0 + e;
        float u = a.bias ? a.bias[d] : 0.0f;
#pragma unroll
        for (int j = 0; j < H; ++j) {
            const long long stream = a.pos - H + j;
            const float past = (stream >= 0 && ring) ? load(ring + ((long long)b * a.D + d) * H + stream % H)
                                                     : 0.0f;
            u = fmaf(a.w[d * W + j], past, u);
        }
        u = fmaf(a.w[d * W + H], xf[e], u);
        h[e] = fmaf(af[e], h[e], (1.0f - af[e]) * u);
        out[e] = h[e];
        if (ring) ring[((long long)b * a.D + d) * H + write_slot] = x[at + e];
    }
    store_raw(static_cast<IO *>(a.y) + at, pack<IO>(out));
    *reinterpret_cast<float4 *>(hstate + at) = make_float4(h[0], h[1], h[2], h[3]);
}

std::atomic<unsigned> g_epoch{0};

template <typename IO>
int scan_typed(const DiagArgs &a, void *ws, size_t bytes, hipStream_t stream) {
    const Layout lay = layout(a.B, a.T, a.D, VEC, sizeof(IO));
    if (bytes < lay.total) return fail(MIRA_ERR_ARG, "diag: workspace too small");
    unsigned epoch = (g_epoch.fetch_add(1) + 1) & 0x3fffffffu;
    if (epoch == 0) epoch = (g_epoch.fetch_add(1) + 1) & 0x3fffffffu;
    const long long blocks = lay.chains * lay.tiles;
    hipLaunchKernelGGL((diag_scan_kernel<IO, 4>), dim3(blocks), dim3(64), 0, stream, a,
                       static_cast<unsigned char *>(ws), epoch);
    return check_launch("diag_scan");
}

template <typename IO>
int step_typed(const DiagArgs &a, float *h, hipStream_t stream) {
    const long long threads = (long long)a.B * (a.D / VEC);
    hipLaunchKernelGGL((diag_step_kernel<IO, 4>), dim3((threads + 255) / 256), dim3(256), 0,
                       stream, a, h);
    return check_launch("diag_step");
}

int vec_of(int) { return VEC; }

}  // namespace

size_t diag_workspace(int B, int T, int D, int dtype) {
    return layout(B, T, D, vec_of(dtype), dtype == MIRA_F32 ? 4 : 2).total;
}

int diag_scan_launch(const DiagArgs &a, void *ws, size_t bytes, hipStream_t stream) {
    switch (a.dtype) {
        case MIRA_F32: return scan_typed<float>(a, ws, bytes, stream);
        case MIRA_BF16: return scan_typed<bf16_t>(a, ws, bytes, stream);
        case MIRA_F16: return scan_typed<f16_t>(a, ws, bytes, stream);
    }
    return fail(MIRA_DECLINE, "diag: unsupported dtype");
}

int diag_step_launch(const DiagArgs &a, float *h, hipStream_t stream) {
    switch (a.dtype) {
        case MIRA_F32: return step_typed<float>(a, h, stream);
        case MIRA_BF16: return step_typed<bf16_t>(a, h, stream);
        case MIRA_F16: return step_typed<f16_t>(a, h, stream);
    }
    return fail(MIRA_DECLINE, "diag: unsupported dtype");
}

int diag_read_error(void *ws, size_t bytes, unsigned *value) {
    if (!ws || bytes < 4) return fail(MIRA_ERR_ARG, "diag: no workspace");
    if (hipMemcpy(value, ws, sizeof(unsigned), hipMemcpyDeviceToHost) != hipSuccess)
        return fail(MIRA_ERR_HIP, "diag: reading the watchdog word failed");
    return MIRA_OK;
}

}  // namespace mira
