// Depthwise causal conv (width W) + diagonal decay scan, prefill and decode, on gfx950.
//
//     u_t = sum_j w[d,j] x_(t-W+1+j) + bias[d],     h_t = a_t h_(t-1) + (1 - a_t) u_t,     y_t = h_t
//
// PREFILL IS ONE PASS OVER HBM. The work is cut into tiles of TILE_T tokens x 256 channels of one
// sequence; the tiles of one (sequence, channel block) -- a chain -- are joined by a decoupled
// look-back over their affine maps h_in -> A h_in + H (A = prod a, H the state reached from
// zero): every tile publishes its aggregate (A, H) as soon as it is known, folds its
// predecessors' aggregates back to the nearest published inclusive state, and publishes its own
// inclusive state. x and a are read once and y written once: 6 bytes per (b, t, d) in bf16.
//
// A WORKGROUP IS ONE LOOK-BACK WAVE AND S STREAMING WAVES, persistent over the tiles it draws from
// its chain's counter. A streaming wave owns TPW consecutive tokens x 256 channels of a tile
// (64 lanes x 4 channels: one 512-byte row piece per access in bf16) and runs a three-stage
// pipeline: it issues the loads of tile i+1, computes the map of tile i (keeping b_t = (1-a_t) u_t
// in LDS), and, after one barrier, replays tile i-1 (h = a h + b) from the entering state the
// look-back wave resolved meanwhile and stores y.
// The look-back wave does all the cross-workgroup protocol (publish, poll, fold, publish), so
// the streaming waves never wait behind its polls: a wave's vector memory operations complete
// in issue order, and a poll issued by a streaming wave would wait for its own prefetch. The
// barriers fence only LDS, never outstanding global loads.
//
// Forward progress: tickets are drawn in chain order, a look-back wave resolves its tiles in
// ticket order, and a tile only waits on lower tickets, so the lowest unresolved tile always
// progresses; the waits are nevertheless bounded, and a wait that runs out sets the workspace's
// watchdog word. Counters return to zero at the end of every launch; flags carry a per-launch
// epoch, so the workspace needs zero-filling only once, when it is allocated.
#include "mira_device.hpp"
#include "mira_abi_internal.hpp"

#include <algorithm>
#include <type_traits>
#include <atomic>

namespace mira {
namespace {

constexpr int VEC = 4;            // channels per lane
constexpr int STREAMS = 7;        // streaming waves per workgroup (plus one look-back wave)
constexpr int TILE_C = 64 * VEC;  // channels per tile
constexpr int WINDOW = 4;         // predecessors the look-back inspects per round
constexpr unsigned SPIN_LIMIT = 1u << 20;
constexpr unsigned OUT_OF_RANGE = 0x80000000u;   // a buffer offset past every record
constexpr int NT = 2;             // non-temporal cache policy for the a stream and y

// tokens per streaming wave and tile: 8 of a 16-bit type (8-byte packs), 4 of float32 (16-byte
// packs), so a lane holds 16 registers of x and 16 of a per tile either way
__host__ __device__ constexpr int tokens_per_wave(int element_bytes) {
    return element_bytes == 4 ? 4 : 8;
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <typename IO> struct Raw { typedef u32x2 type; };
template <> struct Raw<float> { typedef u32x4 type; };

// a buffer resource over one sequence's [T, D] rows (raw addressing, 32-bit offsets)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t resource(const void *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

template <typename IO, int POLICY = 0>
__device__ __forceinline__ typename Raw<IO>::type load_pack(__amdgpu_buffer_rsrc_t r, unsigned off) {
    if constexpr (sizeof(IO) == 4) return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POLICY);
    else return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POLICY);
}

template <typename IO, int POLICY = 0>
__device__ __forceinline__ void store_pack(__amdgpu_buffer_rsrc_t r, unsigned off,
                                           const typename Raw<IO>::type &v) {
    if constexpr (sizeof(IO) == 4) __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, POLICY);
    else __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, POLICY);
}

__device__ __forceinline__ float low_half(unsigned w, bf16_t) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float high_half(unsigned w, bf16_t) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float low_half(unsigned w, f16_t) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
}
__device__ __forceinline__ float high_half(unsigned w, f16_t) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
}

template <typename IO>
__device__ __forceinline__ void unpack(const typename Raw<IO>::type &p, float (&f)[VEC]) {
    if constexpr (sizeof(IO) == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(p[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            f[2 * i] = low_half(p[i], IO{});
            f[2 * i + 1] = high_half(p[i], IO{});
        }
    }
}

template <typename IO>
__device__ __forceinline__ typename Raw<IO>::type pack(const float (&f)[VEC]) {
    typename Raw<IO>::type p;
    if constexpr (sizeof(IO) == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = __float_as_uint(f[i]);
    } else if constexpr (__is_same(IO, bf16_t)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const f32x2 v = {f[2 * i], f[2 * i + 1]};
            p[i] = __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const f32x2 v = {f[2 * i], f[2 * i + 1]};
            p[i] = __builtin_bit_cast(unsigned, __builtin_convertvector(v, f16x2));
        }
    }
    return p;
}

// PUBLICATION WITHOUT AN L2 WRITE-BACK. A release fence at agent scope writes back the whole L2
// of the issuing XCD, so the published records are instead written and read with agent-scope
// relaxed atomics, which go to the device coherence point instead of the XCD's non-coherent L2;
// the writer waits for its record stores to complete (vmcnt(0)) before it stores the flag, and a
// reader loads a record only after it has seen the flag.
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
// | aggregates (A,H)[chains*tiles][VEC][64 lanes] | inclusive H[chains*tiles][VEC][64 lanes]
// (records lane-minor, so a wave's record accesses are contiguous and coalesce)
struct Layout {
    long long chains, tiles, tile_c;
    size_t counters, flags, agg, inc, total;
};

__host__ __device__ inline Layout layout(int B, int T, int D, int element_bytes) {
    Layout l;
    const int tile_t = STREAMS * tokens_per_wave(element_bytes);
    l.tile_c = TILE_C;
    l.chains = (long long)B * ((D + l.tile_c - 1) / l.tile_c);
    l.tiles = (T + tile_t - 1) / tile_t;
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    l.counters = 256;
    l.flags = l.counters + up(l.chains * 4);
    l.agg = l.flags + up(l.chains * l.tiles * 4);
    l.inc = l.agg + up(l.chains * l.tiles * l.tile_c * 8);
    l.total = l.inc + up(l.chains * l.tiles * l.tile_c * 4);
    return l;
}

// LDS-only fences around a barrier: they order LDS accesses and wait for nothing else, so a
// wave's outstanding global loads stay in flight across the barrier
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename IO, int W>
__global__ __launch_bounds__((STREAMS + 1) * 64) __attribute__((amdgpu_waves_per_eu(2)))
void diag_scan_kernel(DiagArgs a, unsigned char *ws, unsigned epoch, int groups_per_chain) {
    constexpr int TPW = tokens_per_wave(sizeof(IO));
    constexpr int TILE_T = STREAMS * TPW;
    constexpr int H = W - 1;                         // conv history
    typedef typename Raw<IO>::type RawT;
    const Layout lay = layout(a.B, a.T, a.D, sizeof(IO));
    unsigned *watchdog = reinterpret_cast<unsigned *>(ws);
    unsigned *counters = reinterpret_cast<unsigned *>(ws + lay.counters);
    unsigned *flags = reinterpret_cast<unsigned *>(ws + lay.flags);
    float2 *agg = reinterpret_cast<float2 *>(ws + lay.agg);
    float *inc = reinterpret_cast<float *>(ws + lay.inc);

    __shared__ int s_ticket[4];                      // tickets t_i, ring of four
    // the streaming waves' maps of tile i, by i mod 3; once the look-back wave has folded them,
    // the same slot carries each wave's resolved entering state (.x)
    __shared__ float2 s_map[3][STREAMS][VEC][64];

    // the wave index as a scalar, so the role branch and per-wave loops are uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int chain = blockIdx.x % lay.chains;
    const int cblocks = (a.D + TILE_C - 1) / TILE_C;
    const int b = chain / cblocks;
    const int d0 = (chain % cblocks) * TILE_C + lane * VEC;
    const bool dact = d0 < a.D;
    const long long row0 = (long long)b * a.T;
    const unsigned tag = (epoch & 0x3fffffffu) << 2;
    const unsigned tag_agg = tag | 1u, tag_inc = tag | 2u;           // flag values
    const unsigned last_draw = (unsigned)lay.tiles + 3u * (unsigned)groups_per_chain - 1u;

    if (wave == 0) {
        // ------------------------------------------------------------------ the look-back wave
        // Tickets are drawn three tiles ahead (a streaming wave reads t_(i+1) before barrier
        // X_i, and the look-back wave writes it between X_(i-2) and X_(i-1)). Each workgroup
        // therefore draws exactly three tickets past the last tile, so the counter's last draw
        // is tiles + 3 groups - 1 and the workgroup that draws it resets the counter.
        auto draw = [&]() -> int {
            unsigned ticket = 0;
            if (lane == 0) {
                ticket = atomicAdd(counters + chain, 1u);
                if (ticket == last_draw)
                    __hip_atomic_store(counters + chain, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return (int)__shfl(ticket, 0);
        };
        const int t0 = draw(), t1 = draw(), t2 = draw();
        if (lane == 0) { s_ticket[0] = t0; s_ticket[1] = t1; s_ticket[2] = t2; }
        lds_barrier();                                               // P
        // the inclusive state of this workgroup's last resolved tile, which its look-backs use
        // without waiting for its flag
        long long own_tile = -1;
        float own_inc[VEC] = {0.0f, 0.0f, 0.0f, 0.0f};
        // the look-back of one tile, WINDOW predecessors per round (lane j < WINDOW polls
        // base - j): folds published aggregates back to the nearest inclusive state
        // `first` is the caller's read of the first round's flags (lane j: tile - 1 - j)
        auto resolve = [&](int tile, float (&hin)[VEC], unsigned first) {
            float cA[VEC], cH[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) { cA[e] = 1.0f; cH[e] = 0.0f; hin[e] = 0.0f; }
            long long base = tile - 1;
            unsigned spins = 0;
            bool fresh = true;
            while (true) {
                unsigned status = 2;                                 // before the first tile
                if (lane < WINDOW && base - lane >= 0) {
                    const unsigned f = fresh ? first
                                             : __hip_atomic_load(flags + (long long)chain * lay.tiles + base - lane,
                                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    status = (f & ~3u) == tag ? (f & 3u) : 0u;
                    if (base - lane == own_tile) status = 2;         // known here, flag or not
                }
                fresh = false;
                const unsigned long long ready = __ballot(lane < WINDOW && status >= 1);
                const unsigned long long inclusive = __ballot(lane < WINDOW && status == 2);
                const int first_inclusive = inclusive ? __builtin_ctzll(inclusive) : WINDOW;
                const unsigned long long need = (1ull << first_inclusive) - 1ull;
                if ((ready & need) != need) {
                    if (++spins > SPIN_LIMIT) {
                        if (lane == 0)
                            __hip_atomic_store(watchdog, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                    continue;
                }
                // the records, nearest first: aggregates, then the inclusive state
                const int count = first_inclusive < WINDOW ? first_inclusive + 1 : WINDOW;
                float2 rec[WINDOW][VEC];
#pragma unroll
                for (int g = 0; g < WINDOW; ++g) {
                    if (g < count) {
                        const long long record = ((long long)chain * lay.tiles + base - g) * TILE_C + lane;
#pragma unroll
                        for (int e = 0; e < VEC; ++e)
                            rec[g][e] = g < first_inclusive ? read_pair(agg + record + e * 64)
                                      : base - g == own_tile ? make_float2(0.0f, own_inc[e])
                                                             : make_float2(0.0f, read_value(inc + record + e * 64));
                    }
                }
#pragma unroll
                for (int g = 0; g < WINDOW; ++g) {
                    if (g < count) {
#pragma unroll
                        for (int e = 0; e < VEC; ++e) {
                            if (g < first_inclusive) {               // fold one more aggregate
                                cH[e] = fmaf(cA[e], rec[g][e].y, cH[e]);
                                cA[e] *= rec[g][e].x;
                            } else {                                 // the inclusive state
                                hin[e] = fmaf(cA[e], rec[g][e].y, cH[e]);
                            }
                        }
                    }
                }
                if (first_inclusive < WINDOW) break;
                base -= WINDOW;
            }
        };
        // the inclusive state of `tile` (map At, Ht; entering state hin) to its record, and each
        // streaming wave's entering state, carried through the maps of the waves before it, to
        // the .x of the tile's map slot `ring` (read after a later barrier)
        auto finish_tile = [&](int tile, int ring, const float (&At)[VEC], const float (&Ht)[VEC],
                               float (&hin)[VEC]) {
            const long long slot = (long long)chain * lay.tiles + tile;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                own_inc[e] = fmaf(At[e], hin[e], Ht[e]);
                publish_value(inc + (slot * VEC + e) * 64 + lane, own_inc[e]);
            }
            own_tile = tile;
#pragma unroll
            for (int g = 0; g < STREAMS; ++g) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float2 m = s_map[ring][g][e][lane];
                    s_map[ring][g][e][lane].x = hin[e];
                    hin[e] = fmaf(m.x, hin[e], m.y);
                }
            }
        };
        // Tile i's aggregate is published after barrier X_i; the tile is resolved one iteration
        // later, after X_(i+1), when the aggregates of the tiles the other workgroups of the chain
        // drew meanwhile are out too, so a look-back rarely waits. Tile 0 needs no look-back and
        // is resolved at once. The streaming waves replay tile i after X_(i+2).
        // The ticket draw is issued first, so its round trip overlaps the others.
        // Iteration i takes barrier X_i while tile i, i - 1 or i - 2 is one of this workgroup's
        // tiles -- the streaming waves run the same count.
        int tile_prev = lay.tiles, tile_prev2 = lay.tiles;           // tiles i - 1, i - 2
        int announce = lay.tiles;                                    // inclusive written, flag pending
        float Ap[VEC], Hp[VEC];                                      // tile i - 1's map
        for (int i = 0;; ++i) {
            // tickets rise, so once a drawn tile is past the end every later one is too
            const int tile = (i == 0 || tile_prev < lay.tiles) ? s_ticket[i & 3] : lay.tiles;
            if (tile >= lay.tiles && tile_prev >= lay.tiles && tile_prev2 >= lay.tiles) break;
            lds_barrier();                                           // X_i: maps of tile i
            const bool live = tile < lay.tiles;
            unsigned drawn = 0;
            if (live && lane == 0) drawn = atomicAdd(counters + chain, 1u);
            float At[VEC], Ht[VEC];
            if (live) {
                // the tile's map: the streaming waves' maps in token order
#pragma unroll
                for (int e = 0; e < VEC; ++e) { At[e] = 1.0f; Ht[e] = 0.0f; }
#pragma unroll
                for (int g = 0; g < STREAMS; ++g) {
#pragma unroll
                    for (int e = 0; e < VEC; ++e) {
                        const float2 m = s_map[i % 3][g][e][lane];
                        Ht[e] = fmaf(m.x, Ht[e], m.y);
                        At[e] *= m.x;
                    }
                }
            }
            // this tile's records go out first; the first look-back poll is issued behind them, so
            // one wait covers both round trips (and the inclusive records of the tile resolved in
            // the previous iteration, whose flag is set now)
            if (live) {
                if (tile == 0) {
                    float hin[VEC];
#pragma unroll
                    for (int e = 0; e < VEC; ++e)
                        hin[e] = (dact && a.h0) ? a.h0[(long long)b * a.D + d0 + e] : 0.0f;
                    finish_tile(0, i % 3, At, Ht, hin);
                } else {
                    const long long slot = (long long)chain * lay.tiles + tile;
#pragma unroll
                    for (int e = 0; e < VEC; ++e)
                        publish_pair(agg + (slot * VEC + e) * 64 + lane, At[e], Ht[e]);
                }
            }
            const bool resolving = tile_prev < lay.tiles && tile_prev != 0;
            unsigned first = 0;
            if (resolving && lane < WINDOW && tile_prev - 1 - lane >= 0)
                first = __hip_atomic_load(flags + (long long)chain * lay.tiles + tile_prev - 1 - lane,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            stores_complete();
            if (lane == 0) {
                if (announce < lay.tiles) set_flag(flags + (long long)chain * lay.tiles + announce, tag_inc);
                if (live) {
                    set_flag(flags + (long long)chain * lay.tiles + tile, tile == 0 ? tag_inc : tag_agg);
                    if (drawn == last_draw)
                        __hip_atomic_store(counters + chain, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    s_ticket[(i + 3) & 3] = (int)drawn;
                }
            }
            announce = lay.tiles;
            if (resolving) {
                float hin[VEC];
                resolve(tile_prev, hin, first);
                finish_tile(tile_prev, (i + 2) % 3, Ap, Hp, hin);
                announce = tile_prev;                                // flag set after the next wait
            }
            if (live) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) { Ap[e] = At[e]; Hp[e] = Ht[e]; }
            }
            tile_prev2 = tile_prev;
            tile_prev = tile;
        }
        if (announce < lay.tiles) {
            stores_complete();
            if (lane == 0) set_flag(flags + (long long)chain * lay.tiles + announce, tag_inc);
        }
        return;
    }

    // -------------------------------------------------------------------- a streaming wave
    const int sw = wave - 1;                                         // token group of the tile
    const unsigned seq_bytes = (unsigned)a.T * (unsigned)a.D * (unsigned)sizeof(IO);
    const IO *x = static_cast<const IO *>(a.x);
    const __amdgpu_buffer_rsrc_t xr = resource(x + row0 * a.D, seq_bytes);
    const __amdgpu_buffer_rsrc_t ar = resource(static_cast<const IO *>(a.a) + row0 * a.D, seq_bytes);
    const __amdgpu_buffer_rsrc_t yr = resource(static_cast<IO *>(a.y) + row0 * a.D, seq_bytes);
    auto offset = [&](int t) -> unsigned {
        return (dact && t >= 0 && t < a.T)
                   ? ((unsigned)t * (unsigned)a.D + (unsigned)d0) * (unsigned)sizeof(IO)
                   : OUT_OF_RANGE;
    };
    float wv[VEC][W], bias[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
#pragma unroll
        for (int j = 0; j < W; ++j) wv[e][j] = dact ? a.w[(long long)(d0 + e) * W + j] : 0.0f;
        bias[e] = (dact && a.bias) ? a.bias[d0 + e] : 0.0f;
    }
    // the H x tokens before token t (the conv history), as raw packs of x; before the first
    // token of this call they come from the ring, or are zero
    auto history = [&](int t, RawT (&hist)[H]) {
#pragma unroll
        for (int j = 0; j < H; ++j) {
            const int tt = t - H + j;
            if (tt >= 0 || !a.ring_in) {
                hist[j] = load_pack<IO>(xr, offset(tt));
            } else {
                float f[VEC] = {0.0f, 0.0f, 0.0f, 0.0f};
                const long long stream = a.pos + tt;
                if (dact && stream >= 0) {
                    const IO *ring = static_cast<const IO *>(a.ring_in);
                    const int s = (int)(stream % H);
#pragma unroll
                    for (int e = 0; e < VEC; ++e) f[e] = load(ring + ((long long)b * a.D + d0 + e) * H + s);
                }
                hist[j] = pack<IO>(f);
            }
        }
    };
    auto fetch = [&](int tile, RawT (&xp)[TPW], RawT (&ap)[TPW], RawT (&hist)[H]) {
        const int t0 = tile * TILE_T + sw * TPW;
        const bool live = tile < lay.tiles;
        if (live) history(t0, hist);
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            const unsigned off = live ? offset(t0 + k) : OUT_OF_RANGE;
            xp[k] = load_pack<IO>(xr, off);
            ap[k] = load_pack<IO, NT>(ar, off);
        }
    };
    // the conv and the decay input of one token: u = w . (x_(t-3), .., x_t) + bias,
    // b = (1 - a) u; `win` holds the H previous x and is shifted
    auto token_input = [&](const float (&xf)[VEC], const float (&af)[VEC], float (&win)[H][VEC],
                           float (&bv)[VEC]) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            float u = bias[e];
#pragma unroll
            for (int j = 0; j < H; ++j) u = fmaf(wv[e][j], win[j][e], u);
            u = fmaf(wv[e][H], xf[e], u);
            bv[e] = fmaf(-af[e], u, u);
#pragma unroll
            for (int j = 0; j + 1 < H; ++j) win[j][e] = win[j + 1][e];
            win[H - 1][e] = xf[e];
        }
    };
    // first pass: conv and decay over the wave's tokens from zero, giving the wave's map (A, H)
    auto summarise = [&](const RawT (&xp)[TPW], const RawT (&ap)[TPW], const RawT (&hist)[H],
                         float (&A)[VEC], float (&h)[VEC]) {
        float win[H][VEC];
#pragma unroll
        for (int j = 0; j < H; ++j) unpack<IO>(hist[j], win[j]);
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            float xf[VEC], af[VEC], bv[VEC];
            unpack<IO>(xp[k], xf);
            unpack<IO>(ap[k], af);
            token_input(xf, af, win, bv);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                h[e] = fmaf(af[e], h[e], bv[e]);
                A[e] *= af[e];
            }
        }
    };
    // second pass: the same tokens from the wave's entering state, recomputing b (bitwise as in
    // the first pass), storing y
    auto replay = [&](int t0, const RawT (&xp)[TPW], const RawT (&ap)[TPW], const RawT (&hist)[H],
                      float (&h)[VEC]) {
        float win[H][VEC];
#pragma unroll
        for (int j = 0; j < H; ++j) unpack<IO>(hist[j], win[j]);
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            float xf[VEC], af[VEC], bv[VEC];
            unpack<IO>(xp[k], xf);
            unpack<IO>(ap[k], af);
            token_input(xf, af, win, bv);
#pragma unroll
            for (int e = 0; e < VEC; ++e) h[e] = fmaf(af[e], h[e], bv[e]);
            store_pack<IO, NT>(yr, offset(t0 + k), pack<IO>(h));
            if (dact && t0 + k == a.T - 1 && a.hT) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) a.hT[(long long)b * a.D + d0 + e] = h[e];
            }
        }
    };

    lds_barrier();                                                   // P
    // Step i: issue tile i+1's loads, summarise tile i, barrier X_i, replay tile i-2 (resolved by
    // the look-back wave after X_(i-1)). Four register sets rotate, so loads land directly in the
    // registers they are used from and a tile's packs stay until its replay (no b buffer in LDS).
    struct Packs { RawT x[TPW], a[TPW], h[H]; };
    Packs set0, set1, set2, set3;
    int tile_cur = s_ticket[0], tile_prev = lay.tiles, tile_prev2 = lay.tiles;
    fetch(tile_cur, set0.x, set0.a, set0.h);
    auto step = [&](int i, Packs &cur, Packs &next, Packs &old) -> bool {
        // the look-back wave runs the same rule, so both take the same barriers
        if (tile_cur >= lay.tiles && tile_prev >= lay.tiles && tile_prev2 >= lay.tiles) return false;
        const int tile_next = tile_cur < lay.tiles ? s_ticket[(i + 1) & 3] : lay.tiles;
        fetch(tile_next, next.x, next.a, next.h);
        if (tile_cur < lay.tiles) {
            float A[VEC] = {1.0f, 1.0f, 1.0f, 1.0f}, Hs[VEC] = {0.0f, 0.0f, 0.0f, 0.0f};
            summarise(cur.x, cur.a, cur.h, A, Hs);
#pragma unroll
            for (int e = 0; e < VEC; ++e) s_map[i % 3][sw][e][lane] = make_float2(A[e], Hs[e]);
        }
        lds_barrier();                                               // X_i
        if (tile_prev2 < lay.tiles) {
            // this wave's entering state in tile i - 2, resolved by the look-back wave
            float h[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) h[e] = s_map[(i + 1) % 3][sw][e][lane].x;
            replay(tile_prev2 * TILE_T + sw * TPW, old.x, old.a, old.h, h);
            // the ring after this call: the last H stream tokens, each in slot (stream mod H)
            if (a.ring_out && tile_prev2 == lay.tiles - 1 && sw == 0 && dact) {
                const IO *ring_in = static_cast<const IO *>(a.ring_in);
                IO *ring_out = static_cast<IO *>(a.ring_out);
#pragma unroll
                for (int j = 0; j < H; ++j) {
                    const long long stream = a.pos + a.T - H + j;
                    const long long t = a.T - H + j;
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
        tile_prev2 = tile_prev;
        tile_prev = tile_cur;
        tile_cur = tile_next;
        return true;
    };
    for (int i = 0;; i += 4) {
        if (!step(i, set0, set1, set2)) break;
        if (!step(i + 1, set1, set2, set3)) break;
        if (!step(i + 2, set2, set3, set0)) break;
        if (!step(i + 3, set3, set0, set1)) break;
    }
}

// one decode token: thread per VEC channels of one sequence. With ALIGNED (ring 8-byte, w and
// bias 16-byte aligned) a thread's ring history (VEC x H values), conv weights (VEC x W) and bias
// are read as whole vectors: 8 loads instead of 32 scalar ones.
template <typename IO, int W, bool ALIGNED>
__global__ __launch_bounds__(256) void diag_step_kernel(DiagArgs a, float *hstate) {
    constexpr int H = W - 1;
    typedef typename Raw<IO>::type RawT;
    const long long index = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long per_row = a.D / VEC;
    if (index >= (long long)a.B * per_row) return;
    const int b = index / per_row;
    const int d0 = (index % per_row) * VEC;
    const IO *x = static_cast<const IO *>(a.x);
    IO *ring = static_cast<IO *>(a.ring_out);
    const long long at = (long long)b * a.D + d0;
    float xf[VEC], af[VEC], h[VEC];
    const RawT xraw = *reinterpret_cast<const RawT *>(x + at);
    unpack<IO>(xraw, xf);
    unpack<IO>(*reinterpret_cast<const RawT *>(static_cast<const IO *>(a.a) + at), af);
    {
        const float4 v = *reinterpret_cast<const float4 *>(hstate + at);
        h[0] = v.x; h[1] = v.y; h[2] = v.z; h[3] = v.w;
    }
    // the ring's H past tokens (slot = stream index mod H), conv weights and bias of VEC channels
    float past[VEC][H], wv[VEC][W], bias[VEC];
    u32x2 r[3] = {};
    if constexpr (ALIGNED && sizeof(IO) == 2 && VEC * H == 12 && W == 4) {
        const unsigned *rw = reinterpret_cast<const unsigned *>(ring + at * H);
        if (ring) {
#pragma unroll
            for (int q = 0; q < 3; ++q) r[q] = reinterpret_cast<const u32x2 *>(rw)[q];
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e)
#pragma unroll
            for (int j = 0; j < H; ++j) {
                const long long stream = a.pos - H + j;
                const int i = e * H + (int)(((stream % H) + H) % H);   // u16 index within 12
                const unsigned word = r[i >> 2][(i >> 1) & 1];
                past[e][j] = (stream >= 0 && ring) ? ((i & 1) ? high_half(word, IO{}) : low_half(word, IO{}))
                                                   : 0.0f;
            }
        const float4 *w4 = reinterpret_cast<const float4 *>(a.w + (long long)d0 * W);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const float4 v = w4[e];
            wv[e][0] = v.x; wv[e][1] = v.y; wv[e][2] = v.z; wv[e][3] = v.w;
        }
        const float4 bv = a.bias ? *reinterpret_cast<const float4 *>(a.bias + d0) : make_float4(0, 0, 0, 0);
        bias[0] = bv.x; bias[1] = bv.y; bias[2] = bv.z; bias[3] = bv.w;
    } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const long long d = d0 + e;
            bias[e] = a.bias ? a.bias[d] : 0.0f;
#pragma unroll
            for (int j = 0; j < W; ++j) wv[e][j] = a.w[d * W + j];
#pragma unroll
            for (int j = 0; j < H; ++j) {
                const long long stream = a.pos - H + j;
                past[e][j] = (stream >= 0 && ring) ? load(ring + ((long long)b * a.D + d) * H + stream % H) : 0.0f;
            }
        }
    }
    const int write_slot = (int)(a.pos % H);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        float u = bias[e];
#pragma unroll
        for (int j = 0; j < H; ++j) u = fmaf(wv[e][j], past[e][j], u);
        u = fmaf(wv[e][H], xf[e], u);
        h[e] = fmaf(af[e], h[e], (1.0f - af[e]) * u);
    }
    if constexpr (ALIGNED && sizeof(IO) == 2 && VEC * H == 12 && W == 4) {
        // the new token goes into its slot of the loaded ring words, which go back whole: three
        // 8-byte stores per 4 channels instead of four 2-byte ones
        if (ring) {
            unsigned word[6] = {r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1]};
            auto put = [&](auto slot) {
                constexpr int S = decltype(slot)::value;
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const int i = e * H + S;
                    const unsigned half = (xraw[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                    word[i >> 1] = (i & 1) ? ((word[i >> 1] & 0xffffu) | (half << 16))
                                           : ((word[i >> 1] & 0xffff0000u) | half);
                }
            };
            if (write_slot == 0) put(std::integral_constant<int, 0>{});
            else if (write_slot == 1) put(std::integral_constant<int, 1>{});
            else put(std::integral_constant<int, 2>{});
            u32x2 *dst = reinterpret_cast<u32x2 *>(ring + at * H);
            dst[0] = u32x2{word[0], word[1]};
            dst[1] = u32x2{word[2], word[3]};
            dst[2] = u32x2{word[4], word[5]};
        }
    } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
            if (ring) ring[(at + e) * H + write_slot] = x[at + e];
    }
    *reinterpret_cast<RawT *>(static_cast<IO *>(a.y) + at) = pack<IO>(h);
    *reinterpret_cast<float4 *>(hstate + at) = make_float4(h[0], h[1], h[2], h[3]);
}

// ---------------------------------------------------------------------------------------------
// column prefill: one workgroup per (sequence, 64-channel column), all T tokens in order
// ---------------------------------------------------------------------------------------------
constexpr int COL_C = 64;                        // channels per column
constexpr int COL_WAVES = 16;
constexpr int COL_SEG = 4;                       // tokens per segment (half a wave)
constexpr int COL_SEGS = 2 * COL_WAVES;          // segments per tile
constexpr int COL_TILE = COL_SEGS * COL_SEG;     // tokens per tile
// tiles whose loads are in flight ahead of use: two of a 16-bit type, one of float32 (whose
// packs are twice the registers)
__host__ __device__ constexpr int col_ahead(int element_bytes) { return element_bytes == 4 ? 1 : 2; }
constexpr int COL_FOLD = 8;                      // maps the folding wave reads per LDS round

// two channels of one token: a dword of a 16-bit type, two of float32
template <typename IO> struct Duo { typedef unsigned type; };
template <> struct Duo<float> { typedef u32x2 type; };

template <typename IO, int POLICY = 0>
__device__ __forceinline__ typename Duo<IO>::type load_duo(__amdgpu_buffer_rsrc_t r, unsigned off) {
    if constexpr (sizeof(IO) == 4) return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POLICY);
    else return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POLICY);
}
template <typename IO, int POLICY = 0>
__device__ __forceinline__ void store_duo(__amdgpu_buffer_rsrc_t r, unsigned off,
                                          const typename Duo<IO>::type &v) {
    if constexpr (sizeof(IO) == 4) __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, POLICY);
    else __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, POLICY);
}
template <typename IO>
__device__ __forceinline__ void unpack_duo(const typename Duo<IO>::type &p, float (&f)[2]) {
    if constexpr (sizeof(IO) == 4) { f[0] = __uint_as_float(p[0]); f[1] = __uint_as_float(p[1]); }
    else { f[0] = low_half(p, IO{}); f[1] = high_half(p, IO{}); }
}
template <typename IO>
__device__ __forceinline__ typename Duo<IO>::type pack_duo(const float (&f)[2]) {
    if constexpr (sizeof(IO) == 4) {
        return u32x2{__float_as_uint(f[0]), __float_as_uint(f[1])};
    } else if constexpr (__is_same(IO, bf16_t)) {
        return __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2{f[0], f[1]}), bf16x2));
    } else {
        return __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2{f[0], f[1]}), f16x2));
    }
}

// THE COLUMN FORM. Where the batch has enough 64-channel columns to give every CU one, a
// workgroup scans its column over all T tokens and no state crosses workgroups. A tile is 128
// tokens: 16 waves x 2 half-wave segments of 4 tokens; a lane holds 2 channels of its segment.
// Step i issues the loads of tile i+2, computes tile i's conv inputs b = (1-a)u and each
// segment's map (A, H) (kept: a and b in registers, the map in LDS), and after one barrier
// wave 0 folds the 32 maps of tile i in token order from the state entering the tile, writing
// each segment's entering state to LDS and carrying the state on to tile i+1, while every wave
// replays tile i-1 (h = a h + b) from the entering states folded in step i-1 and stores y.
template <typename IO, int W>
__global__ __launch_bounds__(COL_WAVES * 64) void diag_column_kernel(DiagArgs a) {
    constexpr int H = W - 1;                     // conv history
    typedef typename Duo<IO>::type DuoT;
    constexpr int AHEAD = col_ahead(sizeof(IO));
    __shared__ alignas(16) float2 s_map[2][COL_SEGS][COL_C];    // each segment's map (A, H), per channel
    __shared__ alignas(16) float s_enter[2][COL_SEGS][COL_C];   // each segment's entering state

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int seg = 2 * wave + (lane >> 5), pair = lane & 31;
    const int columns = (a.D + COL_C - 1) / COL_C;
    const int b = blockIdx.x / columns, c0 = (blockIdx.x % columns) * COL_C;
    const int d = c0 + 2 * pair;                 // this lane's channels d, d + 1 (D is even)
    const bool dact = d < a.D;
    const int tiles = (a.T + COL_TILE - 1) / COL_TILE;
    const long long row0 = (long long)b * a.T;
    const unsigned seq_bytes = (unsigned)a.T * (unsigned)a.D * (unsigned)sizeof(IO);
    const IO *x = static_cast<const IO *>(a.x);
    const __amdgpu_buffer_rsrc_t xr = resource(x + row0 * a.D, seq_bytes);
    const __amdgpu_buffer_rsrc_t ar = resource(static_cast<const IO *>(a.a) + row0 * a.D, seq_bytes);
    const __amdgpu_buffer_rsrc_t yr = resource(static_cast<IO *>(a.y) + row0 * a.D, seq_bytes);
    // Offsets need no range checks: a token at or past T, or before 0 (the 32-bit offset wraps),
    // lies outside the sequence's buffer resource, whose loads read zero and whose stores are
    // dropped; a lane past D starts at OUT_OF_RANGE, and OUT_OF_RANGE + T D bytes < 2^32.
    // offset(tile, k): token tile * COL_TILE + seg * COL_SEG + k (k may be negative); the
    // tile- and k-dependent part is uniform, so each offset is one add to the lane's base.
    const unsigned row_bytes = (unsigned)a.D * (unsigned)sizeof(IO);
    const unsigned lane_base = (dact ? (unsigned)d * (unsigned)sizeof(IO) : OUT_OF_RANGE)
                             + (unsigned)(seg * COL_SEG) * row_bytes;
    auto offset = [&](int tile, int k) -> unsigned {
        return lane_base + (unsigned)(tile * COL_TILE + k) * row_bytes;
    };
    float wv[2][W], bias[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
#pragma unroll
        for (int j = 0; j < W; ++j) wv[e][j] = dact ? a.w[(long long)(d + e) * W + j] : 0.0f;
        bias[e] = (dact && a.bias) ? a.bias[d + e] : 0.0f;
    }
    // the lane, tile and token holding token T - 1 (for the final state)
    const int last_tile = (a.T - 1) / COL_TILE, last_k = (a.T - 1) % COL_SEG;
    const bool holds_last = dact && seg == ((a.T - 1) % COL_TILE) / COL_SEG;

    // raw packs of one tile (x, a and the H x before the segment), loaded AHEAD tiles ahead
    struct Packs { DuoT x[COL_SEG], a[COL_SEG], h[H]; };
    // a tile's decay factors and conv inputs, kept from its summary to its replay
    struct Kept { float a[COL_SEG][2], b[COL_SEG][2]; };
    // the packs of a tile; `first` for tile 0, whose history may come from the ring
    auto fetch = [&](Packs &p, int tile, bool first) {
        const int t0 = tile * COL_TILE + seg * COL_SEG;
#pragma unroll
        for (int j = 0; j < H; ++j) {
            const int tt = t0 - H + j;
            if (!first || tt >= 0 || !a.ring_in) {
                p.h[j] = load_duo<IO>(xr, offset(tile, j - H));
            } else {                             // before this call's first token: the ring
                float f[2] = {0.0f, 0.0f};
                const long long stream = a.pos + tt;
                if (dact && stream >= 0) {
                    const IO *ring = static_cast<const IO *>(a.ring_in);
                    const int s = (int)(stream % H);
#pragma unroll
                    for (int e = 0; e < 2; ++e) f[e] = load(ring + ((long long)b * a.D + d + e) * H + s);
                }
                p.h[j] = pack_duo<IO>(f);
            }
        }
#pragma unroll
        for (int k = 0; k < COL_SEG; ++k) {
            const unsigned off = offset(tile, k);
            p.x[k] = load_duo<IO>(xr, off);
            p.a[k] = load_duo<IO>(ar, off);
        }
    };
    // conv and decay inputs of a segment from zero state, and the segment's map
    auto summarise = [&](const Packs &p, Kept &kept, int ring) {
        float win[H][2];
#pragma unroll
        for (int j = 0; j < H; ++j) unpack_duo<IO>(p.h[j], win[j]);
        float A[2] = {1.0f, 1.0f}, Hs[2] = {0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < COL_SEG; ++k) {
            float xf[2], af[2];
            unpack_duo<IO>(p.x[k], xf);
            unpack_duo<IO>(p.a[k], af);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                float u = bias[e];
#pragma unroll
                for (int j = 0; j < H; ++j) u = fmaf(wv[e][j], win[j][e], u);
                u = fmaf(wv[e][H], xf[e], u);
                const float bv = fmaf(-af[e], u, u);
                kept.a[k][e] = af[e];
                kept.b[k][e] = bv;
                Hs[e] = fmaf(af[e], Hs[e], bv);
                A[e] *= af[e];
#pragma unroll
                for (int j = 0; j + 1 < H; ++j) win[j][e] = win[j + 1][e];
                win[H - 1][e] = xf[e];
            }
        }
        *reinterpret_cast<float4 *>(&s_map[ring][seg][2 * pair]) = make_float4(A[0], Hs[0], A[1], Hs[1]);
    };
    // wave 0, lane = channel: the entering state of every segment of a tile, in token order
    float carry = (lane < COL_C && c0 + lane < a.D && a.h0 && wave == 0) ? a.h0[(long long)b * a.D + c0 + lane]
                                                                        : 0.0f;
    auto fold = [&](int ring) {
#pragma unroll
        for (int s0 = 0; s0 < COL_SEGS; s0 += COL_FOLD) {
            float2 m[COL_FOLD];
#pragma unroll
            for (int s = 0; s < COL_FOLD; ++s) m[s] = s_map[ring][s0 + s][lane];
#pragma unroll
            for (int s = 0; s < COL_FOLD; ++s) {
                s_enter[ring][s0 + s][lane] = carry;
                carry = fmaf(m[s].x, carry, m[s].y);
            }
        }
    };
    auto replay = [&](int tile, const Kept &kept, int ring) {
        const float2 enter = *reinterpret_cast<const float2 *>(&s_enter[ring][seg][2 * pair]);
        float h[2] = {enter.x, enter.y}, hl[2] = {0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < COL_SEG; ++k) {
#pragma unroll
            for (int e = 0; e < 2; ++e) h[e] = fmaf(kept.a[k][e], h[e], kept.b[k][e]);
            store_duo<IO, NT>(yr, offset(tile, k), pack_duo<IO>(h));
            if (k == last_k) { hl[0] = h[0]; hl[1] = h[1]; }
        }
        if (tile == last_tile && a.hT && holds_last) {
            a.hT[(long long)b * a.D + d] = hl[0];
            a.hT[(long long)b * a.D + d + 1] = hl[1];
        }
    };

    // step i: loads of tile i + AHEAD, summary of tile i, barrier, fold of tile i (wave 0),
    // replay of tile i - 1. AHEAD + 1 pack sets and 2 kept sets rotate through unrolled steps.
    // (The early exits between steps matter: a loop that always runs whole groups of steps was
    // compiled with a full wait for outstanding loads inside it and ran 13% slower.)
    auto step = [&](int i, Packs &cur, Packs &ahead, Kept &now, Kept &before) {
        fetch(ahead, i + AHEAD, false);
        if (i < tiles) summarise(cur, now, i & 1);
        lds_barrier();
        if (wave == 0 && i < tiles) fold(i & 1);
        if (i >= 1) replay(i - 1, before, (i - 1) & 1);
    };
    Kept k0, k1;
    if constexpr (AHEAD == 2) {
        Packs p0, p1, p2;
        fetch(p0, 0, true);
        fetch(p1, 1, false);
        for (int i = 0; i <= tiles; i += 6) {
            step(i, p0, p2, k0, k1);
            if (i + 1 > tiles) break;
            step(i + 1, p1, p0, k1, k0);
            if (i + 2 > tiles) break;
            step(i + 2, p2, p1, k0, k1);
            if (i + 3 > tiles) break;
            step(i + 3, p0, p2, k1, k0);
            if (i + 4 > tiles) break;
            step(i + 4, p1, p0, k0, k1);
            if (i + 5 > tiles) break;
            step(i + 5, p2, p1, k1, k0);
        }
    } else {
        static_assert(AHEAD == 1, "one or two tiles ahead");
        Packs p0, p1;
        fetch(p0, 0, true);
        for (int i = 0; i <= tiles; i += 2) {
            step(i, p0, p1, k0, k1);
            if (i + 1 > tiles) break;
            step(i + 1, p1, p0, k1, k0);
        }
    }

    // the ring after this call: the last H stream tokens, each in slot (stream mod H)
    if (a.ring_out && wave == 0 && lane < 32 && dact) {
        const IO *ring_in = static_cast<const IO *>(a.ring_in);
        IO *ring_out = static_cast<IO *>(a.ring_out);
#pragma unroll
        for (int j = 0; j < H; ++j) {
            const long long stream = a.pos + a.T - H + j;
            const long long t = a.T - H + j;
            const int s = (int)(((stream % H) + H) % H);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const long long at = ((long long)b * a.D + d + e) * H + s;
                if (stream < 0) ring_out[at] = from_float<IO>(0.0f);
                else if (t >= 0) ring_out[at] = x[(row0 + t) * a.D + d + e];
                else if (!ring_in) ring_out[at] = from_float<IO>(0.0f);
                else if (ring_in != ring_out) ring_out[at] = ring_in[at];
            }
        }
    }
}

std::atomic<unsigned> g_epoch{0};

// compute units of the current device (cached per device)
int compute_units() {
    static int cached[64] = {0};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
    if (!cached[device]) {
        int count = 0;
        if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess
            || count <= 0)
            count = 256;
        cached[device] = count;
    }
    return cached[device];
}

template <typename IO>
int scan_typed(const DiagArgs &a, void *ws, size_t bytes, hipStream_t stream) {
    const Layout lay = layout(a.B, a.T, a.D, sizeof(IO));
    if (bytes < lay.total) return fail(MIRA_ERR_ARG, "diag: workspace too small");
    if ((unsigned long long)a.T * a.D * sizeof(IO) >= OUT_OF_RANGE)
        return fail(MIRA_DECLINE, "diag: one sequence must hold under 2 GiB of x");
    // the column form wherever the batch has a 64-channel column for at least half the CUs
    // (its offsets run to T + 4 tiles of rows past the sequence start and must not wrap)
    const long long columns = (long long)a.B * ((a.D + COL_C - 1) / COL_C);
    const bool offsets_fit = ((unsigned long long)a.T + 4 * COL_TILE) * a.D * sizeof(IO) < OUT_OF_RANGE;
    if (2 * columns >= compute_units() && offsets_fit) {
        hipLaunchKernelGGL((diag_column_kernel<IO, 4>), dim3(columns), dim3(COL_WAVES * 64), 0, stream, a);
        return check_launch("diag_column");
    }
    // The look-back form tags its flags with a per-launch epoch passed as an argument, so a
    // graph replay would reuse a captured epoch and could read a previous replay's records:
    // refuse capture rather than risk a silently wrong prefill.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone)
        return fail(MIRA_ERR_ARG, "diag: the look-back prefill (batches with fewer 64-channel "
                                  "columns than half the CUs) cannot be captured in a HIP graph");
    unsigned epoch = (g_epoch.fetch_add(1) + 1) & 0x3fffffffu;
    if (epoch == 0) epoch = (g_epoch.fetch_add(1) + 1) & 0x3fffffffu;
    // persistent workgroups: one per CU in all, spread evenly over the chains
    const long long target = 1LL * compute_units();
    const int groups_per_chain = (int)std::max<long long>(
        1, std::min<long long>(lay.tiles, (target + lay.chains - 1) / lay.chains));
    const long long blocks = lay.chains * groups_per_chain;
    hipLaunchKernelGGL((diag_scan_kernel<IO, 4>), dim3(blocks), dim3((STREAMS + 1) * 64), 0,
                       stream, a, static_cast<unsigned char *>(ws), epoch, groups_per_chain);
    return check_launch("diag_scan");
}

template <typename IO>
int step_typed(const DiagArgs &a, float *h, hipStream_t stream) {
    const long long threads = (long long)a.B * (a.D / VEC);
    const auto aligned = [](const void *p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; };
    if (aligned(a.ring_out, 8) && aligned(a.w, 16) && aligned(a.bias, 16))
        hipLaunchKernelGGL((diag_step_kernel<IO, 4, true>), dim3((threads + 255) / 256), dim3(256), 0,
                           stream, a, h);
    else
        hipLaunchKernelGGL((diag_step_kernel<IO, 4, false>), dim3((threads + 255) / 256), dim3(256), 0,
                           stream, a, h);
    return check_launch("diag_step");
}

}  // namespace

size_t diag_workspace(int B, int T, int D, int dtype) {
    return layout(B, T, D, dtype == MIRA_F32 ? 4 : 2).total;
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
