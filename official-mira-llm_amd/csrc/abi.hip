// The C-ABI of libmira_hip.so (declared in include/mira_hip.h): argument checks, error codes and
// the dispatch to the kernel launchers. Nothing here allocates device memory: workspaces come
// from the caller.
#include "mira_device.hpp"
#include "mira_abi_internal.hpp"

#include <algorithm>
#include <mutex>
#include <string>

namespace mira {

namespace {
thread_local std::string g_last_error;

// The static scratch of mira_lattice_forward_static: one array per GPU (each device holds its
// own copy at its own address), resolved once per device by hipGetSymbolAddress. Host code only
// ever passes the resolved device address; the array's name is a host-side stand-in.
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[MIRA_LATTICE_STATIC_SCRATCH_BYTES];
std::mutex g_scratch_lock;
void *g_scratch[kMaxDevices] = {};

int static_scratch(void **address) {
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices)
        return fail(MIRA_ERR_HIP, "mira: no current HIP device for the static scratch");
    std::lock_guard<std::mutex> hold(g_scratch_lock);
    if (!g_scratch[device]) {
        void *resolved = nullptr;
        const hipError_t status = hipGetSymbolAddress(&resolved, HIP_SYMBOL(scratch));
        if (status != hipSuccess || !resolved)
            return fail(MIRA_ERR_HIP, std::string("mira: hipGetSymbolAddress(scratch) failed: ") +
                                          hipGetErrorString(status));
        g_scratch[device] = resolved;
    }
    *address = g_scratch[device];
    return MIRA_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

int fail(int code, const std::string &message) {
    g_last_error = message;
    return code;
}

int check_launch(const char *what) {
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess)
        return fail(MIRA_ERR_HIP, std::string(what) + ": " + hipGetErrorString(status));
    return MIRA_OK;
}

}  // namespace mira

using namespace mira;

extern "C" {

const char *mira_last_error(void) { return g_last_error.c_str(); }

#ifndef MIRA_SOURCE_HASH
#define MIRA_SOURCE_HASH "unknown"
#endif
const char *mira_version(void) { return "mira_hip 0.1 gfx950 src:" MIRA_SOURCE_HASH; }

int mira_lattice_supported(int K, int M, int dtype) { return lattice_supported(K, M, dtype) ? 1 : 0; }

int mira_lattice_plan_chunk(int B, int T, int C, int K, int M) {
    if (B <= 0 || T <= 0 || C <= 0 || K <= 0 || M <= 0) return 0;
    return lattice_plan_chunk(B, T, C, K, M);
}

size_t mira_lattice_workspace_bytes(int B, int T, int C, int K, int M, int chunk) {
    if (B <= 0 || T <= 0 || C <= 0 || K <= 0 || M <= 0) return 0;
    if (chunk <= 0) chunk = lattice_plan_chunk(B, T, C, K, M);
    return lattice_workspace(B, T, C, K, M, chunk);
}

static int lattice_common(LatticeArgs &a, int64_t x_row, int64_t alpha_row, int64_t beta_row,
                          int64_t rho_row, int64_t gamma_row, int64_t read_row) {
    if (a.B <= 0 || a.T <= 0 || a.C <= 0)
        return fail(MIRA_ERR_ARG, "mira: requires nonempty batch, token and channel axes");
    if (!lattice_supported(a.K, a.M, a.dtype))
        return fail(MIRA_DECLINE, "mira: no kernel for K=" + std::to_string(a.K) +
                                      " d_m=" + std::to_string(a.M) +
                                      " dtype=" + std::to_string(a.dtype));
    if (!arch_valid(a.mode)) return fail(MIRA_ERR_ARG, "mira: unknown arch mode");
    if (!a.x || !a.alpha || !a.beta || !a.rho || !a.gamma || !a.write || !a.read || !a.out)
        return fail(MIRA_ERR_ARG, "mira: a required tensor is null");
    if (x_row < a.C || gamma_row < a.C || alpha_row < (int64_t)a.C * a.K ||
        beta_row < (int64_t)a.C * a.K || rho_row < (int64_t)a.C * (a.K + 1) ||
        read_row < (int64_t)(a.K + 1) * a.M)
        return fail(MIRA_DECLINE, "mira: a row stride is narrower than its row");
    if (a.state_out && a.state_in && a.state_out == a.state_in && a.T > 1)
        return fail(MIRA_ERR_ARG, "mira: state_out may not alias state_in over several tokens");
    a.x_row = x_row; a.alpha_row = alpha_row; a.beta_row = beta_row; a.rho_row = rho_row;
    a.gamma_row = gamma_row; a.read_row = read_row;
    return MIRA_OK;
}

int mira_lattice_forward(const void *x, int64_t x_row, const void *alpha, int64_t alpha_row,
                         const void *beta, int64_t beta_row, const void *rho, int64_t rho_row,
                         const void *gamma, int64_t gamma_row, const void *memory_write,
                         const void *memory_read, int64_t read_row, const uint8_t *valid,
                         const float *state_in, float *state_out, void *out, int B, int T, int C,
                         int K, int M, int dtype, int arch_mode, int chunk, void *workspace,
                         size_t workspace_bytes, void *stream) {
    LatticeArgs a{};
    a.x = x; a.alpha = alpha; a.beta = beta; a.rho = rho; a.gamma = gamma;
    a.write = memory_write; a.read = memory_read; a.valid = valid;
    a.state_in = state_in; a.state_out = state_out; a.out = out;
    a.B = B; a.T = T; a.C = C; a.K = K; a.M = M; a.dtype = dtype; a.mode = arch_mode;
    if (int rc = lattice_common(a, x_row, alpha_row, beta_row, rho_row, gamma_row, read_row))
        return rc;
    if (chunk <= 0) chunk = lattice_plan_chunk(B, T, C, K, M);
    if (chunk > T) chunk = T;
    a.chunk = chunk;
    a.chunks = (T + chunk - 1) / chunk;
    const size_t need = lattice_workspace(B, T, C, K, M, chunk);
    if (need > 0) {
        if (!workspace || workspace_bytes < need)
            return fail(MIRA_ERR_ARG, "mira: workspace smaller than mira_lattice_workspace_bytes");
        const long long planes = (long long)B * a.chunks * C;
        a.phi = static_cast<float *>(workspace);
        a.carry = a.phi + planes * K * K;
    }
    return lattice_launch(a, static_cast<hipStream_t>(stream));
}

int mira_lattice_forward_static(const void *x, int64_t x_row, const void *alpha,
                                int64_t alpha_row, const void *beta, int64_t beta_row,
                                const void *rho, int64_t rho_row, const void *gamma,
                                int64_t gamma_row, const void *memory_write,
                                const void *memory_read, int64_t read_row, const uint8_t *valid,
                                const float *state_in, float *state_out, void *out, int B, int T,
                                int C, int K, int M, int dtype, int arch_mode, int chunk,
                                void *stream) {
    LatticeArgs a{};
    a.x = x; a.alpha = alpha; a.beta = beta; a.rho = rho; a.gamma = gamma;
    a.write = memory_write; a.read = memory_read; a.valid = valid;
    a.state_in = state_in; a.state_out = state_out; a.out = out;
    a.B = B; a.T = T; a.C = C; a.K = K; a.M = M; a.dtype = dtype; a.mode = arch_mode;
    if (int rc = lattice_common(a, x_row, alpha_row, beta_row, rho_row, gamma_row, read_row))
        return rc;
    if (chunk <= 0) chunk = lattice_plan_chunk(B, T, C, K, M);
    if (chunk > T) chunk = T;
    a.chunk = chunk;
    a.chunks = (T + chunk - 1) / chunk;
    const size_t need = lattice_workspace(B, T, C, K, M, chunk);
    if (need > MIRA_LATTICE_STATIC_SCRATCH_BYTES)
        return fail(MIRA_ERR_ARG, "mira: this call's chunk summaries need " + std::to_string(need) +
                                      " bytes, over the " +
                                      std::to_string(MIRA_LATTICE_STATIC_SCRATCH_BYTES) +
                                      "-byte static scratch; pass a longer chunk or use "
                                      "mira_lattice_forward with a workspace");
    if (need > 0) {
        void *base = nullptr;
        if (int rc = static_scratch(&base)) return rc;
        const long long planes = (long long)B * a.chunks * C;
        a.phi = static_cast<float *>(base);
        a.carry = a.phi + planes * K * K;
    }
    return lattice_launch(a, static_cast<hipStream_t>(stream));
}

int mira_lattice_backward_chunk(int K, int M) { return lattice_backward_chunk(K, M); }

size_t mira_lattice_backward_workspace_bytes(int B, int T, int C, int K, int M) {
    if (B <= 0 || T <= 0 || C <= 0 || K <= 0 || M <= 0) return 0;
    return lattice_backward_workspace(B, T, C, K, M);
}

int mira_lattice_backward(const void *x, int64_t x_row, const void *alpha, int64_t alpha_row,
                          const void *beta, int64_t beta_row, const void *rho, int64_t rho_row,
                          const void *gamma, int64_t gamma_row, const void *memory_write,
                          const void *memory_read, int64_t read_row, const uint8_t *valid,
                          const float *state_in, const void *grad_out, void *grad_x,
                          int64_t grad_x_row, void *grad_alpha, int64_t grad_alpha_row,
                          void *grad_beta, int64_t grad_beta_row, void *grad_rho,
                          int64_t grad_rho_row, void *grad_gamma, int64_t grad_gamma_row,
                          void *grad_write, int64_t grad_write_row, const void *raw_write,
                          int64_t raw_write_row, void *grad_read, int64_t grad_read_row, int B,
                          int T, int C, int K, int M, int dtype, int arch_mode,
                          const void *forward_workspace, size_t forward_workspace_bytes,
                          void *workspace, size_t workspace_bytes, void *stream) {
    LatticeArgs f{};
    f.x = x; f.alpha = alpha; f.beta = beta; f.rho = rho; f.gamma = gamma;
    f.write = memory_write; f.read = memory_read; f.out = const_cast<void *>(grad_out);
    f.B = B; f.T = T; f.C = C; f.K = K; f.M = M; f.dtype = dtype; f.mode = arch_mode;
    if (int rc = lattice_common(f, x_row, alpha_row, beta_row, rho_row, gamma_row, read_row))
        return rc;
    const int chunk = lattice_backward_chunk(K, M);
    if (!chunk)
        return fail(MIRA_DECLINE, "mira: no backward kernel for K=" + std::to_string(K) +
                                      " d_m=" + std::to_string(M));
    if (!grad_x || !grad_alpha || !grad_beta || !grad_rho || !grad_gamma || !grad_write ||
        !grad_read)
        return fail(MIRA_ERR_ARG, "mira: a gradient output is null");
    if (grad_x_row < C || grad_gamma_row < C || grad_alpha_row < (int64_t)C * K ||
        grad_beta_row < (int64_t)C * K || grad_rho_row < (int64_t)C * (K + 1) ||
        grad_write_row < M || grad_read_row < (int64_t)(K + 1) * M ||
        (raw_write && raw_write_row < M))
        return fail(MIRA_ERR_ARG, "mira: a gradient row stride is narrower than its row");
    LatticeBackArgs a{};
    a.x = x; a.x_row = x_row; a.alpha = alpha; a.alpha_row = alpha_row; a.beta = beta;
    a.beta_row = beta_row; a.rho = rho; a.rho_row = rho_row; a.gamma = gamma;
    a.gamma_row = gamma_row; a.write = memory_write; a.read = memory_read; a.read_row = read_row;
    a.valid = valid; a.state_in = state_in; a.grad_out = grad_out;
    a.grad_x = grad_x; a.grad_x_row = grad_x_row; a.grad_alpha = grad_alpha;
    a.grad_alpha_row = grad_alpha_row; a.grad_beta = grad_beta; a.grad_beta_row = grad_beta_row;
    a.grad_rho = grad_rho; a.grad_rho_row = grad_rho_row; a.grad_gamma = grad_gamma;
    a.grad_gamma_row = grad_gamma_row; a.grad_write = grad_write;
    a.grad_write_row = grad_write_row; a.raw_write = raw_write; a.raw_write_row = raw_write_row;
    a.grad_read = grad_read; a.grad_read_row = grad_read_row;
    a.B = B; a.T = T; a.C = C; a.K = K; a.M = M; a.dtype = dtype; a.mode = arch_mode;
    a.chunk = chunk;
    a.chunks = (T + chunk - 1) / chunk;
    if (a.chunks > 1) {
        const size_t need = lattice_workspace(B, T, C, K, M, chunk);
        if (!forward_workspace || forward_workspace_bytes < need)
            return fail(MIRA_ERR_ARG, "mira: the backward needs the workspace of a forward run at "
                                      "mira_lattice_backward_chunk's chunk length");
        const long long planes = (long long)B * a.chunks * C;
        a.phi = static_cast<const float *>(forward_workspace);
        a.entering = a.phi + planes * K * K;
    }
    const size_t need = lattice_backward_workspace(B, T, C, K, M);
    if (!workspace || workspace_bytes < need)
        return fail(MIRA_ERR_ARG, "mira: workspace smaller than mira_lattice_backward_workspace_bytes");
    if (reinterpret_cast<uintptr_t>(workspace) % 16)
        return fail(MIRA_ERR_ARG, "mira: the backward workspace must be 16-byte aligned");
    float *base = static_cast<float *>(workspace);
    a.adjoint = a.chunks > 1 ? base : nullptr;
    a.partial = base + (a.chunks > 1 ? (long long)B * a.chunks * C * K * M : 0);
    return lattice_backward_launch(a, static_cast<hipStream_t>(stream));
}

int mira_lattice_step(const void *x, int64_t x_row, const void *alpha, int64_t alpha_row,
                      const void *beta, int64_t beta_row, const void *rho, int64_t rho_row,
                      const void *gamma, int64_t gamma_row, const void *memory_write,
                      const void *memory_read, int64_t read_row, const uint8_t *valid,
                      const float *state_in, float *state_out, void *out, int B, int C, int K,
                      int M, int dtype, int arch_mode, void *stream) {
    LatticeArgs a{};
    a.x = x; a.alpha = alpha; a.beta = beta; a.rho = rho; a.gamma = gamma;
    a.write = memory_write; a.read = memory_read; a.valid = valid;
    a.state_in = state_in; a.state_out = state_out; a.out = out;
    a.B = B; a.T = 1; a.C = C; a.K = K; a.M = M; a.dtype = dtype; a.mode = arch_mode;
    if (int rc = lattice_common(a, x_row, alpha_row, beta_row, rho_row, gamma_row, read_row))
        return rc;
    a.chunk = 1;
    a.chunks = 1;
    return lattice_launch(a, static_cast<hipStream_t>(stream));
}

int mira_lattice_control_serves(int B, int T, int C, int K, int M, int R, int dtype) {
    return lattice_control_serves(B, T, C, K, M, R, dtype) ? 1 : 0;
}

int mira_lattice_control_forward(const void *x, int64_t x_row, const void *control,
                                 const void *weight, int64_t weight_row, int64_t weight_rows,
                                 const void *bias, int64_t alpha_first, int64_t beta_first,
                                 int64_t rho_first, const void *gamma, int64_t gamma_row,
                                 const void *memory_write, const void *memory_read,
                                 int64_t read_row, const uint8_t *valid, const float *state_in,
                                 float *state_out, void *out, int B, int T, int C, int K, int M,
                                 int R, int dtype, int arch_mode, void *stream) {
    if (B <= 0 || T <= 0 || C <= 0 || R <= 0)
        return fail(MIRA_ERR_ARG, "mira: requires nonempty batch, token, channel and control axes");
    if (!arch_valid(arch_mode)) return fail(MIRA_ERR_ARG, "mira: unknown arch mode");
    if (!lattice_control_serves(B, T, C, K, M, R, dtype))
        return fail(MIRA_DECLINE, "mira: the control scan serves bf16, (K, d_m) in {(1,8), (1,16), "
                                  "(2,8), (2,16), (4,8)}, d_r in {16,32,48,64} and calls one token "
                                  "chunk covers");
    if (!x || !control || !weight || !gamma || !memory_write || !memory_read || !out)
        return fail(MIRA_ERR_ARG, "mira: a required tensor is null");
    if (x_row < C || gamma_row < C || read_row < (int64_t)(K + 1) * M || weight_row < R)
        return fail(MIRA_DECLINE, "mira: a row stride is narrower than its row");
    if (!aligned16(control) || (reinterpret_cast<uintptr_t>(weight) & 7u) || weight_row % 4 ||
        (reinterpret_cast<uintptr_t>(memory_write) & 3u) ||
        (reinterpret_cast<uintptr_t>(memory_read) & 3u) || read_row % 2)
        return fail(MIRA_DECLINE, "mira: control must be 16-byte aligned, weight rows 8-byte "
                                  "aligned, memory_write and memory_read rows 4-byte aligned");
    const int64_t last = std::max({alpha_first + (int64_t)C * K, beta_first + (int64_t)C * K,
                                   rho_first + (int64_t)C * (K + 1)});
    if (alpha_first < 0 || beta_first < 0 || rho_first < 0 || last > weight_rows)
        return fail(MIRA_ERR_ARG, "mira: coefficient rows fall outside the weight");
    LatticeControlArgs a{};
    a.x = x; a.x_row = x_row; a.control = control; a.weight = weight; a.weight_row = weight_row;
    a.bias = bias; a.alpha_first = alpha_first; a.beta_first = beta_first; a.rho_first = rho_first;
    a.gamma = gamma; a.gamma_row = gamma_row; a.write = memory_write; a.read = memory_read;
    a.read_row = read_row; a.valid = valid; a.state_in = state_in; a.state_out = state_out;
    a.out = out; a.B = B; a.T = T; a.C = C; a.K = K; a.M = M; a.R = R; a.mode = arch_mode;
    return lattice_control_launch(a, static_cast<hipStream_t>(stream));
}

size_t mira_diag_workspace_bytes(int B, int T, int D, int dtype) {
    if (B <= 0 || T <= 0 || D <= 0 || dtype < MIRA_F32 || dtype > MIRA_F16) return 0;
    return diag_workspace(B, T, D, dtype);
}

static int diag_common(const DiagArgs &a) {
    if (a.B <= 0 || a.T <= 0 || a.D <= 0)
        return fail(MIRA_ERR_ARG, "diag: requires nonempty batch, token and channel axes");
    if (a.dtype < MIRA_F32 || a.dtype > MIRA_F16) return fail(MIRA_DECLINE, "diag: unsupported dtype");
    if (a.W != 4) return fail(MIRA_DECLINE, "diag: conv width must be 4");
    const int vec = 4;
    if (a.D % vec) return fail(MIRA_DECLINE, "diag: D must be a multiple of 4");
    if (!a.x || !a.a || !a.w || !a.y) return fail(MIRA_ERR_ARG, "diag: a required tensor is null");
    if (!aligned16(a.x) || !aligned16(a.a) || !aligned16(a.y))
        return fail(MIRA_DECLINE, "diag: x, a and y must be 16-byte aligned");
    if (a.pos < 0) return fail(MIRA_ERR_ARG, "diag: pos must be >= 0");
    return MIRA_OK;
}

int mira_diag_conv_scan(const void *x, const void *a, const float *w, const float *bias,
                        const float *h0, const void *ring_in, void *ring_out, int64_t pos,
                        void *y, float *hT, int B, int T, int D, int W, int dtype,
                        void *workspace, size_t workspace_bytes, void *stream) {
    DiagArgs d{};
    d.x = x; d.a = a; d.w = w; d.bias = bias; d.h0 = h0; d.ring_in = ring_in; d.ring_out = ring_out;
    d.pos = pos; d.y = y; d.hT = hT; d.B = B; d.T = T; d.D = D; d.W = W; d.dtype = dtype;
    if (int rc = diag_common(d)) return rc;
    if (!workspace) return fail(MIRA_ERR_ARG, "diag: workspace is null");
    return diag_scan_launch(d, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int mira_diag_conv_step(const void *x, const void *a, const float *w, const float *bias,
                        float *h, void *ring, int64_t pos, void *y, int B, int D, int W,
                        int dtype, void *stream) {
    DiagArgs d{};
    d.x = x; d.a = a; d.w = w; d.bias = bias; d.ring_in = ring; d.ring_out = ring; d.pos = pos;
    d.y = y; d.B = B; d.T = 1; d.D = D; d.W = W; d.dtype = dtype;
    if (int rc = diag_common(d)) return rc;
    if (!h || !aligned16(h)) return fail(MIRA_ERR_ARG, "diag: h must be a 16-byte aligned state");
    return diag_step_launch(d, h, static_cast<hipStream_t>(stream));
}

int mira_diag_workspace_error(void *workspace, size_t workspace_bytes, unsigned *value) {
    return diag_read_error(workspace, workspace_bytes, value);
}

static int gla_common(const GlaArgs &a) {
    if (a.B <= 0 || a.T <= 0 || a.H <= 0)
        return fail(MIRA_ERR_ARG, "gla: requires nonempty batch, token and head axes");
    if (a.dk != 128 || a.dv != 128) return fail(MIRA_DECLINE, "gla: d_k = d_v = 128 only");
    if (a.dtype < MIRA_F32 || a.dtype > MIRA_F16) return fail(MIRA_DECLINE, "gla: unsupported dtype");
    if (!a.q || !a.k || !a.v || !a.g || !a.o) return fail(MIRA_ERR_ARG, "gla: a required tensor is null");
    if ((a.S0 && !aligned16(a.S0)) || (a.ST && !aligned16(a.ST)))
        return fail(MIRA_DECLINE, "gla: states must be 16-byte aligned");
    return MIRA_OK;
}

size_t mira_gla_workspace_bytes(int B, int T, int H, int dk, int dv) {
    return gla_workspace(B, T, H, dk, dv);
}

int mira_gla_chunked(const void *q, const void *k, const void *v, const float *g,
                     const float *S0, float *ST, void *o, int B, int T, int H, int dk, int dv,
                     int dtype, void *workspace, size_t workspace_bytes, void *stream) {
    GlaArgs a{};
    a.q = q; a.k = k; a.v = v; a.g = g; a.S0 = S0; a.ST = ST; a.o = o;
    a.B = B; a.T = T; a.H = H; a.dk = dk; a.dv = dv; a.dtype = dtype;
    if (int rc = gla_common(a)) return rc;
    if (workspace_bytes < gla_workspace(B, T, H, dk, dv))
        return fail(MIRA_ERR_ARG, "gla: workspace smaller than mira_gla_workspace_bytes");
    return gla_chunked_launch(a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int mira_gla_step(const void *q, const void *k, const void *v, const float *g, float *S,
                  void *o, int B, int H, int dk, int dv, int dtype, void *stream) {
    GlaArgs a{};
    a.q = q; a.k = k; a.v = v; a.g = g; a.S0 = S; a.ST = S; a.o = o;
    a.B = B; a.T = 1; a.H = H; a.dk = dk; a.dv = dv; a.dtype = dtype;
    if (int rc = gla_common(a)) return rc;
    if (!S) return fail(MIRA_ERR_ARG, "gla: the state is null");
    return gla_step_launch(a, static_cast<hipStream_t>(stream));
}

}  // extern "C"
