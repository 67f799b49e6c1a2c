// abi.cpp -- extern "C" entry points of libmi355gemm.so (declared in
// include/mi355_gemm.h).  Validation happens here, before any launch; the
// scheduler resolves the kernel; launches are asynchronous on the caller's
// stream.  Nothing here allocates device memory or keeps state between calls
// other than an immutable per-device CU count.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>

#include "../../include/mi355_gemm.h"
#include "gemm_kernel.hpp"
#include "mi_internal.hpp"

namespace mi {
int validate_shape(const mi_gemm_args& a);
int plan_gemm(const mi_gemm_args& a, int num_cus, mi_plan& out, GemmLaunch* launch);
// the packed N/T problem of a plan with mi_plan.packed (operands in workspace)
mi_gemm_args packed_problem(const mi_gemm_args& a, void* workspace, size_t workspace_bytes);
}  // namespace mi

using namespace mi;

namespace {

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];  // 0 = not queried yet

int device_cus(int* status) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
        *status = MI_ERR_NO_DEVICE;
        return 0;
    }
    if (dev < kMaxDevices) {
        const int cached = g_cu_count[dev].load(std::memory_order_relaxed);
        if (cached > 0) return cached;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
        *status = MI_ERR_NO_DEVICE;
        return 0;
    }
    if (dev < kMaxDevices) g_cu_count[dev].store(n, std::memory_order_relaxed);
    return n;
}

int hip_rc(hipError_t e) { return e == hipSuccess ? MI_OK : (int)e; }

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

mi_gemm_args dense_args(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N,
                        int op_a, int op_b) {
    mi_gemm_args a{};
    a.A = A;
    a.B = B;
    a.C = C;
    a.M = M;
    a.N = N;
    a.K = K;
    a.batch = 1;
    a.op_a = op_a;
    a.op_b = op_b;
    a.lda = op_a == MI_OP_N ? K : M;
    a.ldb = op_b == MI_OP_N ? N : K;
    a.ldc = N;
    a.structure = MI_DENSE;
    return a;
}

// MI_SYMMETRIC is the dense product C = op_a(A) . op_b(B) of square
// operands, computed as given: like kernels/13_...:57,134-151 it does not rely
// on the symmetry, so a non-symmetric input still gets its own product.  (The
// symmetry would allow reading B as stored N x K, but the N/N kernel is the
// faster one at 8192^3: 7.32 vs 7.38 ms.)
// A named dense operator's call: the caller's workspace (NULL: none) bounds
// the plan, as mi_gemm_args.workspace_bytes does.
int run_with_workspace(mi_gemm_args a, void* workspace, size_t workspace_bytes, void* stream);

int canonical(mi_gemm_args& a) {
    if (a.structure != MI_SYMMETRIC) return MI_OK;
    if (a.M != a.N || a.N != a.K) return MI_ERR_NOT_SQUARE;
    a.structure = MI_DENSE;
    return MI_OK;
}

}  // namespace

extern "C" {

const char* mi_status_string(int status) {
    switch (status) {
        case MI_OK: return "ok";
        case MI_ERR_NULL_POINTER: return "null pointer argument";
        case MI_ERR_BAD_SIZE: return "invalid size (negative, or beyond the supported range)";
        case MI_ERR_BAD_LAYOUT: return "invalid op / structure combination";
        case MI_ERR_BAD_LD: return "leading dimension or batch stride too small";
        case MI_ERR_NOT_SQUARE: return "structured (triangular) product needs square operands";
        case MI_ERR_WORKSPACE: return "workspace missing or too small";
        case MI_ERR_NO_DEVICE: return "no HIP device available";
        case MI_ERR_ALIGNMENT: return "pointer not 16-byte aligned";
        case MI_ERR_SCRATCH_LIMIT:
            return "the forced plan needs more scratch than mi_gemm_f32_noalloc's fixed "
                   "64 MiB device array holds (use mi_gemm_f32 with a workspace)";
        default: break;
    }
    if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
    return "unknown status";
}

const char* mi_version(void) { return "mi355_gemm 0.1.0 gfx950"; }

int mi_gemm_plan(const mi_gemm_args* args, int32_t num_cus, mi_plan* out) {
    if (!args || !out) return MI_ERR_NULL_POINTER;
    mi_gemm_args a = *args;
    const int rc = canonical(a);
    if (rc != MI_OK) return rc;
    return plan_gemm(a, num_cus, *out, nullptr);
}

int mi_gemm_tile_of(const mi_gemm_args* args, int32_t num_cus, int64_t item, int32_t split,
                    int32_t* tile_m, int32_t* tile_n, int64_t* k_begin, int64_t* k_end) {
    if (!args || !tile_m || !tile_n || !k_begin || !k_end) return MI_ERR_NULL_POINTER;
    mi_gemm_args ca = *args;
    int rc = canonical(ca);
    if (rc != MI_OK) return rc;
    mi_plan p{};
    GemmLaunch g{};
    rc = plan_gemm(ca, num_cus, p, &g);
    if (rc != MI_OK) return rc;
    // the chunked triangular list (dynamic order) continues past its compute
    // items with the zero tiles its workgroups write
    const int64_t n_items =
        g.num_tiles + (g.tri_cap >= 2 ? tri_zero_items(g.tiles_m, g.tri_cap) : 0);
    if (item < 0 || item >= n_items || split < 0 || split >= g.split_k) return MI_ERR_BAD_SIZE;
    if (g.sk_tiles > 0) return MI_ERR_BAD_LAYOUT;  // stream-K: mi_gemm_work_item
    const GemmParams kp = make_params(g);
    int tm = 0, tn = 0, kb = 0, ke = 0;
    bool compute;
    if (is_panel_cfg(g.cfg)) {
        // panel kernel: tile item = row-major (tm, tn); every tile reduces all of K
        *tile_m = (int32_t)(item / g.tiles_n);
        *tile_n = (int32_t)(item % g.tiles_n);
        *k_begin = 0;
        *k_end = g.K;
        return 1;
    }
    if (g.tri_cap > 0) {
        // chunked triangular list: 2 marks a chunk whose partial sum is
        // stored in the mirror tile (tile_n, tile_m) and added in afterwards;
        // 3 a zero-triangle tile the workgroup writes with +0.0 (no K range)
        if (item >= g.num_tiles) {
            tri_zero_tile((int)(item - g.num_tiles), g.tiles_m, g.structure == kLower, tm, tn);
            *tile_m = tm;
            *tile_n = tn;
            *k_begin = 0;
            *k_end = 0;
            return 3;
        }
        int u0, u1, mirror;
        tri_item((int)item, g.tiles_m, g.tri_cap, g.structure == kLower, tm, tn, u0, u1, mirror);
        *tile_m = tm;
        *tile_n = tn;
        *k_begin = (int64_t)u0 * 256;
        *k_end = std::min<int64_t>(g.K, (int64_t)u1 * 256);
        return mirror ? 2 : 1;
    }
    const int bid = (int)item, nb = g.num_tiles;
#define MI_TILE_OF(BMN)                                                                        \
    (g.structure == kLower  ? tile_of<BMN, BMN, kLower>(kp, bid, nb, split, tm, tn, kb, ke)  \
     : g.structure == kUpper ? tile_of<BMN, BMN, kUpper>(kp, bid, nb, split, tm, tn, kb, ke) \
                             : tile_of<BMN, BMN, kDense>(kp, bid, nb, split, tm, tn, kb, ke))
    switch (g.cfg) {
        case kCfg64:
        case kCfg64W: compute = MI_TILE_OF(64); break;
        case kCfg128:
        case kCfg128W8:
        case kCfg128K32:
        case kCfg128K64:
        case kCfg128B32: compute = MI_TILE_OF(128); break;
        default: compute = MI_TILE_OF(256); break;
    }
#undef MI_TILE_OF
    *tile_m = tm;
    *tile_n = tn;
    *k_begin = kb;
    *k_end = ke;
    return compute ? 1 : 0;
}

int mi_gemm_work_item(const mi_gemm_args* args, int32_t num_cus, int64_t wg, int32_t split,
                      int64_t item, mi_work_item* out) {
    if (!args || !out) return MI_ERR_NULL_POINTER;
    mi_gemm_args ca = *args;
    int rc = canonical(ca);
    if (rc != MI_OK) return rc;
    mi_plan p{};
    GemmLaunch g{};
    rc = plan_gemm(ca, num_cus, p, &g);
    if (rc != MI_OK) return rc;
    if (is_panel_cfg(g.cfg) || g.structure != kDense) return MI_ERR_BAD_LAYOUT;
    if (wg < 0 || wg >= g.grid_x || split < 0 || split >= g.split_k || item < 0) return MI_ERR_BAD_SIZE;
    if (item > INT32_MAX) return 0;
    const CfgInfo ci = cfg_info(g.cfg);
    if (g.sk_tiles > 0) {
        int lt, s0, s1;
        int64_t slot;
        if (!sk_item((int)wg, (int)item, g.grid_x, g.sk_dp, g.sk_tiles, g.sk_ipt, g.sk_ph, g.sk_nph,
                     lt, s0, s1, slot))
            return 0;
        int tm, tn;
        raster(lt, g.tiles_m, g.tiles_n, g.group_m, tm, tn);
        out->tile_m = tm;
        out->tile_n = tn;
        out->k_begin = (int64_t)s0 * ci.bk;
        out->k_end = std::min<int64_t>((int64_t)s1 * ci.bk, g.K);  // (4-byte staging: last slice partial)
        out->dest = slot >= 0 ? 1 : 0;
        out->slot = slot >= 0 ? (int32_t)slot : 0;
        return 1;
    }
    const int64_t t = wg + item * g.grid_x;
    if (t >= g.num_tiles) return 0;
    const GemmParams kp = make_params(g);
    int tm = 0, tn = 0, kb = 0, ke = 0;
    switch (g.cfg) {
        case kCfg64:
        case kCfg64W: tile_of<64, 64, kDense>(kp, (int)t, g.num_tiles, split, tm, tn, kb, ke); break;
        case kCfg256: tile_of<256, 256, kDense>(kp, (int)t, g.num_tiles, split, tm, tn, kb, ke); break;
        case kCfg128B32:
        default: tile_of<128, 128, kDense>(kp, (int)t, g.num_tiles, split, tm, tn, kb, ke); break;
    }
    out->tile_m = tm;
    out->tile_n = tn;
    out->k_begin = kb;
    out->k_end = ke;
    out->dest = g.split_k > 1 ? 1 : 0;
    out->slot = g.split_k > 1 ? split : 0;
    return 1;
}

int mi_gemm_sk_fixup_of(const mi_gemm_args* args, int32_t num_cus, int64_t t, int32_t* tile_m,
                        int32_t* tile_n, int64_t* first_slot, int64_t* n_slots) {
    if (!args || !tile_m || !tile_n || !first_slot || !n_slots) return MI_ERR_NULL_POINTER;
    mi_gemm_args ca = *args;
    int rc = canonical(ca);
    if (rc != MI_OK) return rc;
    mi_plan p{};
    GemmLaunch g{};
    rc = plan_gemm(ca, num_cus, p, &g);
    if (rc != MI_OK) return rc;
    if (g.sk_tiles <= 0) return MI_ERR_BAD_LAYOUT;
    if (t < 0 || t >= g.sk_tiles) return MI_ERR_BAD_SIZE;
    int tm, tn;
    raster(g.sk_dp + (int)t, g.tiles_m, g.tiles_n, g.group_m, tm, tn);
    *tile_m = tm;
    *tile_n = tn;
    sk_tile_slots(t, g.sk_tiles, g.sk_ipt, g.grid_x, g.sk_ph, g.sk_nph, *first_slot, *n_slots);
    return 1;
}

size_t mi_gemm_workspace_bytes(const mi_gemm_args* args) {
    if (!args) return 0;
    mi_gemm_args a = *args;
    if (canonical(a) != MI_OK) return 0;
    a.workspace_bytes = SIZE_MAX;  // ask what the preferred plan wants
    int st = MI_OK;
    const int cus = device_cus(&st);
    mi_plan p{};
    if (plan_gemm(a, st == MI_OK ? cus : 256, p, nullptr) != MI_OK) return 0;
    return p.workspace_bytes;
}

int mi_gemm_f32(const mi_gemm_args* args, void* stream) {
    if (!args) return MI_ERR_NULL_POINTER;
    mi_gemm_args a = *args;
    int rc = canonical(a);
    if (rc != MI_OK) return rc;
    rc = validate_shape(a);
    if (rc != MI_OK) return rc;
    const bool empty_out = a.M == 0 || a.N == 0 || a.batch == 0;
    if (empty_out) return MI_OK;
    if (!a.C) return MI_ERR_NULL_POINTER;
    hipStream_t s = as_stream(stream);
    if (a.K == 0)
        return hip_rc(launch_fill_zero_2d(a.C, a.M, a.N, a.ldc, a.batch, a.stride_c, s, a.bias_m));
    if (!a.A || !a.B) return MI_ERR_NULL_POINTER;

    int st = MI_OK;
    const int cus = device_cus(&st);
    if (st != MI_OK) return st;
    mi_plan p{};
    GemmLaunch g{};
    rc = plan_gemm(a, cus, p, &g);
    if (rc != MI_OK) return rc;
    if (p.packed) {
        // copy both operands K-contiguous into the workspace, K zero-padded,
        // then run the N/T product of the copies (planned without packing)
        if (!a.workspace || a.workspace_bytes < p.workspace_bytes) return MI_ERR_WORKSPACE;
        const mi_gemm_args pa = packed_problem(a, a.workspace, a.workspace_bytes);
        hipError_t e = launch_pack_rows(a.A, a.lda, a.op_a == MI_OP_N, a.M, a.K,
                                        const_cast<float*>(pa.A), pa.K, s);
        if (e == hipSuccess)
            e = launch_pack_rows(a.B, a.ldb, a.op_b == MI_OP_T, a.N, a.K, const_cast<float*>(pa.B),
                                 pa.K, s);
        if (e != hipSuccess) return hip_rc(e);
        return mi_gemm_f32(&pa, stream);
    }
    if ((g.split_k > 1 || g.sk_tiles > 0) &&
        (!a.workspace || a.workspace_bytes < p.workspace_bytes))
        return MI_ERR_WORKSPACE;

    hipError_t e;
    if (a.op_a == MI_OP_N && a.op_b == MI_OP_N) e = launch_gemm_nn(g, s);
    else if (a.op_a == MI_OP_T && a.op_b == MI_OP_N) e = launch_gemm_tn(g, s);
    else if (a.op_a == MI_OP_N && a.op_b == MI_OP_T) e = launch_gemm_nt(g, s);
    else e = launch_gemm_tt(g, s);
    if (e != hipSuccess) return hip_rc(e);
    if (g.split_k > 1)
        e = launch_splitk_reduce(g.ws, a.C, g.M, g.N, g.batch, g.split_k, a.ldc, a.stride_c,
                                 a.bias_m, s);
    return hip_rc(e);
}

// ---- named operators ---------------------------------------------------------
// The dense products take the caller's workspace (NULL: none) and plan within
// it; their *_workspace_bytes queries return what the preferred plan wants.

int mi_square_matmul_f32(const float* A, const float* B, float* C, int64_t N, void* workspace,
                         size_t workspace_bytes, void* stream) {
    mi_gemm_args a = dense_args(A, B, C, N, N, N, MI_OP_N, MI_OP_N);
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

size_t mi_square_matmul_workspace_bytes(int64_t N) {
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, N, N, N, MI_OP_N, MI_OP_N);
    return mi_gemm_workspace_bytes(&a);
}

int mi_matmul_f32(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N,
                  void* workspace, size_t workspace_bytes, void* stream) {
    mi_gemm_args a = dense_args(A, B, C, M, K, N, MI_OP_N, MI_OP_N);
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

size_t mi_matmul_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, M, K, N, MI_OP_N, MI_OP_N);
    return mi_gemm_workspace_bytes(&a);
}

namespace {
mi_gemm_args batched_args(const float* A, const float* B, float* C, int64_t batch, int64_t M,
                          int64_t K, int64_t N) {
    mi_gemm_args a = dense_args(A, B, C, M, K, N, MI_OP_N, MI_OP_N);
    a.batch = batch;
    a.stride_a = M * K;
    a.stride_b = K * N;
    a.stride_c = M * N;
    return a;
}
}  // namespace

int mi_batched_matmul_f32(const float* A, const float* B, float* C, int64_t batch, int64_t M,
                          int64_t K, int64_t N, void* workspace, size_t workspace_bytes,
                          void* stream) {
    return run_with_workspace(batched_args(A, B, C, batch, M, K, N), workspace, workspace_bytes,
                              stream);
}

size_t mi_batched_matmul_workspace_bytes(int64_t batch, int64_t M, int64_t K, int64_t N) {
    mi_gemm_args a = batched_args(nullptr, nullptr, nullptr, batch, M, K, N);
    return mi_gemm_workspace_bytes(&a);
}

size_t mi_gemv_workspace_bytes(int64_t M, int64_t K) {
    if (M <= 0 || K <= 0) return 0;
    return gemv_plan(M, K, true).ws_bytes;
}

int mi_gemv_f32(const float* A, const float* x, float* y, int64_t M, int64_t K, void* workspace,
                size_t workspace_bytes, void* stream) {
    if (M < 0 || K < 0 || M > INT32_MAX || K > INT32_MAX - 1024) return MI_ERR_BAD_SIZE;
    if (M == 0) return MI_OK;
    if (!y) return MI_ERR_NULL_POINTER;
    hipStream_t s = as_stream(stream);
    if (K == 0) return hip_rc(launch_fill_zero_2d(y, 1, M, M, 1, 0, s));
    if (!A || !x) return MI_ERR_NULL_POINTER;
    const bool aligned = K % 4 == 0 && ((uintptr_t)A & 15u) == 0 && ((uintptr_t)x & 15u) == 0;
    GemvPlan p = gemv_plan(M, K, aligned);
    if (p.split_k > 1 && (!workspace || workspace_bytes < p.ws_bytes)) {
        // Not enough scratch for the split: run unsplit (same result order
        // per row is not required -- each split sum is deterministic either way).
        p.split_k = 1;
        p.k_chunk = (int)K;
        p.ws_bytes = 0;
    }
    return hip_rc(launch_gemv(p, A, x, y, static_cast<float*>(workspace), (int)M, (int)K, K, s));
}

size_t mi_matmul_large_k_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, M, K, N, MI_OP_N, MI_OP_N);
    return mi_gemm_workspace_bytes(&a);
}

int mi_matmul_large_k_f32(const float* A, const float* B, float* C, int64_t M, int64_t K,
                          int64_t N, void* workspace, size_t workspace_bytes, void* stream) {
    mi_gemm_args a = dense_args(A, B, C, M, K, N, MI_OP_N, MI_OP_N);
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

int mi_gemm_small_k_f32(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N,
                        void* stream) {
    mi_gemm_args a = dense_args(A, B, C, M, K, N, MI_OP_N, MI_OP_N);
    return mi_gemm_f32(&a, stream);
}

int mi_tall_skinny_matmul_f32(const float* A, const float* B, float* C, int64_t M, int64_t N,
                              void* stream) {
    mi_gemm_args a = dense_args(A, B, C, M, N, M, MI_OP_N, MI_OP_N);
    return mi_gemm_f32(&a, stream);
}

int mi_tensor3d_matmul_f32(const float* A, const float* B, float* out, int64_t N, int64_t M,
                           int64_t K, int64_t L, void* workspace, size_t workspace_bytes,
                           void* stream) {
    if (N < 0 || M < 0) return MI_ERR_BAD_SIZE;
    mi_gemm_args a = dense_args(A, B, out, N * M, K, L, MI_OP_N, MI_OP_N);
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

size_t mi_tensor3d_matmul_workspace_bytes(int64_t N, int64_t M, int64_t K, int64_t L) {
    if (N < 0 || M < 0) return 0;
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, N * M, K, L, MI_OP_N, MI_OP_N);
    return mi_gemm_workspace_bytes(&a);
}

int mi_tensor4d_matmul_f32(const float* A, const float* B, float* out, int64_t b, int64_t i,
                           int64_t j, int64_t l, int64_t k, void* workspace,
                           size_t workspace_bytes, void* stream) {
    if (b < 0 || i < 0 || j < 0) return MI_ERR_BAD_SIZE;
    mi_gemm_args a = dense_args(A, B, out, b * i * j, l, k, MI_OP_N, MI_OP_N);
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

size_t mi_tensor4d_matmul_workspace_bytes(int64_t b, int64_t i, int64_t j, int64_t l, int64_t k) {
    if (b < 0 || i < 0 || j < 0) return 0;
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, b * i * j, l, k, MI_OP_N, MI_OP_N);
    return mi_gemm_workspace_bytes(&a);
}

int mi_diag_mult_f32(const float* a, const float* B, float* out, int64_t N, int64_t M,
                     void* stream) {
    if (N < 0 || M < 0) return MI_ERR_BAD_SIZE;
    if (N == 0 || M == 0) return MI_OK;
    if (!a || !B || !out) return MI_ERR_NULL_POINTER;
    return hip_rc(launch_diag(a, B, out, N, M, as_stream(stream)));
}

int mi_matrix_scalar_mult_f32(const float* A, float* C, int64_t n, float s, void* stream) {
    if (n < 0) return MI_ERR_BAD_SIZE;
    if (n == 0) return MI_OK;
    if (!A || !C) return MI_ERR_NULL_POINTER;
    return hip_rc(launch_scale(A, C, n, s, as_stream(stream)));
}

int mi_pointwise_conv_f32(const float* input, const float* weight, const float* bias,
                          float* output, int64_t batch, int64_t in_channels, int64_t out_channels,
                          int64_t hw, void* stream) {
    if (batch < 0 || in_channels < 0 || out_channels < 0 || hw < 0) return MI_ERR_BAD_SIZE;
    // per image: out (Cout x HW) = W (Cout x Cin) . X (Cin x HW) + bias
    mi_gemm_args a = dense_args(weight, input, output, out_channels, in_channels, hw, MI_OP_N,
                                MI_OP_N);
    a.batch = batch;
    a.stride_a = 0;
    a.stride_b = in_channels * hw;
    a.stride_c = out_channels * hw;
    a.bias_m = bias;
    return mi_gemm_f32(&a, stream);
}

size_t mi_sdpa_workspace_bytes(int64_t batch_heads, int64_t seq, int64_t embed) {
    if (batch_heads <= 0 || seq <= 0 || embed <= 0 || seq > 32768 || embed > 65536) return 0;
    return sdpa_workspace_bytes(batch_heads, (int)seq, (int)embed);
}

int mi_sdpa_f16(const void* Q, const void* K, const void* V, void* O, int64_t batch_heads,
                int64_t seq, int64_t embed, void* workspace, size_t workspace_bytes, void* stream) {
    if (batch_heads < 0 || seq < 0 || embed < 0 || seq > 32768 || embed > 65536)
        return MI_ERR_BAD_SIZE;
    if (batch_heads == 0 || seq == 0 || embed == 0) return MI_OK;
    if (embed % 64 != 0) return MI_ERR_BAD_SIZE;
    if (!Q || !K || !V || !O) return MI_ERR_NULL_POINTER;
    for (const void* p : {Q, K, V, static_cast<const void*>(O)})
        if (((uintptr_t)p & 15u) != 0) return MI_ERR_ALIGNMENT;
    if (!workspace || workspace_bytes < sdpa_workspace_bytes(batch_heads, (int)seq, (int)embed))
        return MI_ERR_WORKSPACE;
    if (((uintptr_t)workspace & 15u) != 0) return MI_ERR_ALIGNMENT;
    return hip_rc(launch_sdpa(static_cast<const _Float16*>(Q), static_cast<const _Float16*>(K),
                              static_cast<const _Float16*>(V), static_cast<_Float16*>(O), batch_heads,
                              (int)seq, (int)embed, workspace, as_stream(stream)));
}

int mi_symmetric_matmul_f32(const float* A, const float* B, float* C, int64_t N, void* workspace,
                            size_t workspace_bytes, void* stream) {
    // C = A . B as given (the dense N/N plan), symmetric or not
    mi_gemm_args a = dense_args(A, B, C, N, N, N, MI_OP_N, MI_OP_N);
    a.structure = MI_SYMMETRIC;
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

size_t mi_symmetric_matmul_workspace_bytes(int64_t N) {
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, N, N, N, MI_OP_N, MI_OP_N);
    a.structure = MI_SYMMETRIC;
    return mi_gemm_workspace_bytes(&a);
}

int mi_upper_tri_matmul_f32(const float* A, const float* B, float* C, int64_t N, void* stream) {
    mi_gemm_args a = dense_args(A, B, C, N, N, N, MI_OP_N, MI_OP_N);
    a.structure = MI_UPPER;
    return mi_gemm_f32(&a, stream);
}

int mi_lower_tri_mul_f32(const float* A, const float* B, float* C, int64_t N, void* stream) {
    mi_gemm_args a = dense_args(A, B, C, N, N, N, MI_OP_N, MI_OP_N);
    a.structure = MI_LOWER;
    return mi_gemm_f32(&a, stream);
}

int mi_matmul_transposed_a_f32(const float* A, const float* B, float* C, int64_t M, int64_t K,
                               int64_t N, void* workspace, size_t workspace_bytes, void* stream) {
    mi_gemm_args a = dense_args(A, B, C, M, K, N, MI_OP_T, MI_OP_N);
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

size_t mi_matmul_transposed_a_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, M, K, N, MI_OP_T, MI_OP_N);
    return mi_gemm_workspace_bytes(&a);
}

int mi_matmul_transposed_b_f32(const float* A, const float* B, float* C, int64_t M, int64_t K,
                               int64_t N, void* workspace, size_t workspace_bytes, void* stream) {
    mi_gemm_args a = dense_args(A, B, C, M, K, N, MI_OP_N, MI_OP_T);
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

size_t mi_matmul_transposed_b_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, M, K, N, MI_OP_N, MI_OP_T);
    return mi_gemm_workspace_bytes(&a);
}

int mi_matmul_transposed_both_f32(const float* A, const float* B, float* C, int64_t M, int64_t K,
                                  int64_t N, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    mi_gemm_args a = dense_args(A, B, C, M, K, N, MI_OP_T, MI_OP_T);
    return run_with_workspace(a, workspace, workspace_bytes, stream);
}

size_t mi_matmul_transposed_both_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    mi_gemm_args a = dense_args(nullptr, nullptr, nullptr, M, K, N, MI_OP_T, MI_OP_T);
    return mi_gemm_workspace_bytes(&a);
}

int mi_fill_uniform_f32(float* out, int64_t n, uint64_t seed, int64_t offset, void* stream) {
    if (n < 0 || offset < 0) return MI_ERR_BAD_SIZE;
    if (n == 0) return MI_OK;
    if (!out) return MI_ERR_NULL_POINTER;
    return hip_rc(launch_fill_uniform(out, n, seed, offset, as_stream(stream)));
}

}  // extern "C"

namespace {
int run_with_workspace(mi_gemm_args a, void* workspace, size_t workspace_bytes, void* stream) {
    a.workspace = workspace;
    a.workspace_bytes = workspace ? workspace_bytes : 0;
    return mi_gemm_f32(&a, stream);
}
}  // namespace
