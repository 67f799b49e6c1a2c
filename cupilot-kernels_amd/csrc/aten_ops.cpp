// aten_ops.cpp -- the drop-in operator layer: one libtorch function per
// reference operator, same name, same (Tensor A, Tensor B) signature, same
// TORCH_CHECK messages where the reference has them, reaching the HIP kernels
// only through the C ABI of include/mi355_gemm.h.
//
// Differences from the reference wrappers, all on purpose:
//   * outputs are allocated with at::empty (every kernel writes every output
//     element, structural zeros included), not torch::zeros;
//   * work is enqueued on the caller's current HIP stream and never
//     synchronises the host (kernels/1_...:207 synchronises the device,
//     kernels/6_...:147-200 creates and joins 8 streams);
//   * dtype / device / shape checks the reference leaves to luck are added, so a
//     bad call raises before any launch instead of reading out of bounds;
//   * transposed views are consumed in place (the layout goes to the kernel as
//     an op flag) instead of being copied.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <string>

#include "../../include/mi355_gemm.h"

namespace mi355 {

namespace {

void* current_stream(const at::Tensor& t) {
    return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_rc(int rc, const char* op) {
    TORCH_CHECK(rc == MI_OK, op, ": ", mi_status_string(rc), " (status ", rc, ")");
}

void check_tensor(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
    TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be float32");
}

void check_same_device(const at::Tensor& a, const at::Tensor& b) {
    TORCH_CHECK(a.device() == b.device(), "A and B must be on the same device");
}

// How a logical rows x cols matrix is held: op N = row-major with row stride
// ld; op T = stored transposed (cols x rows, row stride ld).
struct MatView {
    at::Tensor keep;  // owns a contiguous copy when one was needed
    const float* ptr;
    int op;
    int64_t ld;
};

// `t` is 2-D; `transpose` says the operator consumes t^T.
MatView view_of(const at::Tensor& t, bool transpose) {
    const int64_t rows = transpose ? t.size(1) : t.size(0);
    const int64_t cols = transpose ? t.size(0) : t.size(1);
    const int64_t rs = transpose ? t.stride(1) : t.stride(0);
    const int64_t cs = transpose ? t.stride(0) : t.stride(1);
    if ((cs == 1 || cols <= 1) && rs >= std::max<int64_t>(cols, 1))
        return {at::Tensor(), t.data_ptr<float>(), MI_OP_N, std::max<int64_t>(rs, cols)};
    if ((rs == 1 || rows <= 1) && cs >= std::max<int64_t>(rows, 1))
        return {at::Tensor(), t.data_ptr<float>(), MI_OP_T, std::max<int64_t>(cs, rows)};
    at::Tensor c = (transpose ? t.t() : t).contiguous();
    return {c, c.data_ptr<float>(), MI_OP_N, std::max<int64_t>(cols, 1)};
}

at::Tensor workspace_for(const mi_gemm_args& a, const at::Tensor& like) {
    const size_t bytes = mi_gemm_workspace_bytes(&a);
    if (bytes == 0) return at::Tensor();
    return at::empty({(int64_t)bytes}, like.options().dtype(at::kByte));
}

// C (M x N, fresh) = op(A) . op(B) for 2-D operands given as logical views.
at::Tensor gemm2d(const at::Tensor& A, bool ta, const at::Tensor& B, bool tb, int structure,
                  const char* op) {
    const int64_t M = ta ? A.size(1) : A.size(0);
    const int64_t K = ta ? A.size(0) : A.size(1);
    const int64_t N = tb ? B.size(0) : B.size(1);
    at::Tensor C = at::empty({M, N}, A.options());
    if (M == 0 || N == 0) return C;
    if (K == 0) return C.zero_();
    MatView va = view_of(A, ta), vb = view_of(B, tb);
    // Operands whose rows are not 16-byte aligned (kernels/8_...'s irregular
    // shapes) are used in place: the engine stages them with 4-byte direct
    // loads at the aligned rate (8205 x 5921 x 2949: 126 TFLOP/s).
    mi_gemm_args a{};
    a.A = va.ptr;
    a.B = vb.ptr;
    a.C = C.data_ptr<float>();
    a.M = M;
    a.N = N;
    a.K = K;
    a.batch = 1;
    a.lda = va.ld;
    a.ldb = vb.ld;
    a.ldc = N;
    a.op_a = va.op;
    a.op_b = vb.op;
    a.structure = structure;
    if (structure != MI_DENSE && (a.op_a != MI_OP_N || a.op_b != MI_OP_N)) {
        // triangular kernels read row-major operands
        at::Tensor ca = (ta ? A.t() : A).contiguous(), cb = (tb ? B.t() : B).contiguous();
        va = {ca, ca.data_ptr<float>(), MI_OP_N, K};
        vb = {cb, cb.data_ptr<float>(), MI_OP_N, N};
        a.A = va.ptr;
        a.B = vb.ptr;
        a.lda = K;
        a.ldb = N;
        a.op_a = a.op_b = MI_OP_N;
    }
    at::Tensor ws = workspace_for(a, A);
    if (ws.defined()) {
        a.workspace = ws.data_ptr();
        a.workspace_bytes = (size_t)ws.numel();
    }
    check_rc(mi_gemm_f32(&a, current_stream(A)), op);
    return C;
}

void check_pair(const at::Tensor& A, const at::Tensor& B) {
    check_tensor(A, "A");
    check_tensor(B, "B");
    check_same_device(A, B);
}

}  // namespace

// kernels/1_Square_matrix_multiplication_best_kernel.cu:189-214
at::Tensor square_matmul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    check_pair(A, B);
    const int64_t N = A.size(0);
    if (N == 0) return at::zeros({0, 0}, A.options());
    TORCH_CHECK(A.size(1) == N && B.size(0) == N && B.size(1) == N,
                "A and B must both be N x N with N = A.size(0)");
    return gemm2d(A, false, B, false, MI_DENSE, "matmul_cuda");
}

// kernels/2_Standard_matrix_multiplication_best_kernel.cu:117-140 and
// kernels/8_Matmul_with_irregular_shapes_best_kernel.cu:155-168
at::Tensor matmul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(A.size(1) == B.size(0), "Matrix dimensions do not match");
    check_pair(A, B);
    return gemm2d(A, false, B, false, MI_DENSE, "matmul_cuda");
}

// kernels/3_Batched_matrix_multiplication_best_kernel.cu:113-148
at::Tensor batched_matmul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 3, "A must be 3D tensor");
    TORCH_CHECK(B.dim() == 3, "B must be 3D tensor");
    TORCH_CHECK(A.size(0) == B.size(0), "A and B must have the same batch size");
    TORCH_CHECK(A.size(2) == B.size(1), "A and B inner dimensions do not match");
    check_pair(A, B);
    const int64_t batch = A.size(0), M = A.size(1), K = A.size(2), N = B.size(2);
    at::Tensor C = at::empty({batch, M, N}, A.options());
    if (batch == 0 || M == 0 || N == 0) return C;
    if (K == 0) return C.zero_();
    // Each batch slice must be a plain or transposed matrix with a uniform
    // batch stride; anything else is copied once.
    auto slice_view = [](const at::Tensor& t, int64_t rows, int64_t cols, at::Tensor& keep,
                         int& op, int64_t& ld, int64_t& bstride) -> const float* {
        const int64_t rs = t.stride(1), cs = t.stride(2);
        if ((cs == 1 || cols <= 1) && rs >= std::max<int64_t>(cols, 1)) {
            op = MI_OP_N;
            ld = std::max<int64_t>(rs, cols);
        } else if ((rs == 1 || rows <= 1) && cs >= std::max<int64_t>(rows, 1)) {
            op = MI_OP_T;
            ld = std::max<int64_t>(cs, rows);
        } else {
            keep = t.contiguous();
            op = MI_OP_N;
            ld = std::max<int64_t>(cols, 1);
            bstride = rows * cols;
            return keep.data_ptr<float>();
        }
        bstride = t.size(0) > 1 ? t.stride(0) : 0;
        return t.data_ptr<float>();
    };
    at::Tensor ka, kb;
    mi_gemm_args a{};
    a.A = slice_view(A, M, K, ka, a.op_a, a.lda, a.stride_a);
    a.B = slice_view(B, K, N, kb, a.op_b, a.ldb, a.stride_b);
    a.C = C.data_ptr<float>();
    a.M = M;
    a.N = N;
    a.K = K;
    a.batch = batch;
    a.ldc = N;
    a.stride_c = M * N;
    a.structure = MI_DENSE;
    at::Tensor ws = workspace_for(a, A);
    if (ws.defined()) {
        a.workspace = ws.data_ptr();
        a.workspace_bytes = (size_t)ws.numel();
    }
    check_rc(mi_gemm_f32(&a, current_stream(A)), "batched_matmul_cuda");
    return C;
}

// kernels/4_Matrix_vector_multiplication_best_kernel.cu:84-108
at::Tensor gemv(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    const int64_t M = A.size(0), K = A.size(1);
    TORCH_CHECK(B.size(0) == K, "A and B shapes not matched");
    TORCH_CHECK(B.size(1) == 1, "B must be a column vector");
    check_pair(A, B);
    at::Tensor C = at::empty({M, 1}, A.options());
    if (M == 0) return C;
    if (K == 0) return C.zero_();
    at::Tensor x = B.reshape({K}).contiguous();
    const bool row_major = A.stride(1) == 1 && A.stride(0) >= K;
    if (!row_major && A.stride(0) == 1 && A.stride(1) >= M) {
        // A is a transposed view: y = (A^T stored)^T . x on the contraction engine
        mi_gemm_args a{};
        a.A = A.data_ptr<float>();
        a.B = x.data_ptr<float>();
        a.C = C.data_ptr<float>();
        a.M = M;
        a.N = 1;
        a.K = K;
        a.batch = 1;
        a.lda = A.stride(1);
        a.ldb = 1;
        a.ldc = 1;
        a.op_a = MI_OP_T;
        a.op_b = MI_OP_N;
        at::Tensor ws = workspace_for(a, A);
        if (ws.defined()) {
            a.workspace = ws.data_ptr();
            a.workspace_bytes = (size_t)ws.numel();
        }
        check_rc(mi_gemm_f32(&a, current_stream(A)), "gemv_cuda");
        return C;
    }
    at::Tensor Ac = row_major && A.stride(0) == K ? A : A.contiguous();
    const size_t wsb = mi_gemv_workspace_bytes(M, K);
    at::Tensor ws = wsb ? at::empty({(int64_t)wsb}, A.options().dtype(at::kByte)) : at::Tensor();
    check_rc(mi_gemv_f32(Ac.data_ptr<float>(), x.data_ptr<float>(), C.data_ptr<float>(), M, K,
                         ws.defined() ? ws.data_ptr() : nullptr, wsb, current_stream(A)),
             "gemv_cuda");
    return C;
}

// kernels/6_Matmul_with_large_K_dimension_best_kernel.cu:128-203
at::Tensor matmul_large_k(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(B.size(0) == A.size(1), "Matrix dimensions mismatch");
    check_pair(A, B);
    return gemm2d(A, false, B, false, MI_DENSE, "matmul_cuda");
}

// kernels/7_Matmul_with_small_K_dimension_best_kernel.cu:80-105
at::Tensor gemm_small_k(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(A.size(1) == B.size(0), "Matrix dimensions do not match");
    check_pair(A, B);
    return gemm2d(A, false, B, false, MI_DENSE, "gemm_cuda");
}

// kernels/9_Tall_skinny_matrix_multiplication_best_kernel.cu:145-198
at::Tensor tall_skinny_matmul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(B.size(0) == A.size(1) && B.size(1) == A.size(0),
                "B must be N x M for A of shape M x N");
    check_pair(A, B);
    return gemm2d(A, false, B, false, MI_DENSE, "tall_skinny_matmul_cuda");
}

// kernels/10_3D_tensor_matrix_multiplication_best_kernel.cu:180-209
at::Tensor tensor3d_matmul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 3, "A must be 3D tensor");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(A.size(2) == B.size(0), "A and B inner dimensions do not match");
    check_pair(A, B);
    const int64_t N = A.size(0), M = A.size(1), L = B.size(1);
    at::Tensor A2 = A.reshape({N * M, A.size(2)});  // a view when A's leading dims collapse
    return gemm2d(A2, false, B, false, MI_DENSE, "batched_matmul_cuda").view({N, M, L});
}

// kernels/11_4D_tensor_matrix_multiplication_best_kernel.cu:132-166
at::Tensor tensor4d_matmul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 4, "A must be 4D tensor");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(A.size(3) == B.size(0), "A and B inner dimensions do not match");
    check_pair(A, B);
    const int64_t b = A.size(0), i = A.size(1), j = A.size(2), k = B.size(1);
    at::Tensor A2 = A.reshape({b * i * j, A.size(3)});
    return gemm2d(A2, false, B, false, MI_DENSE, "tensor_matmul_cuda").view({b, i, j, k});
}

// kernels/12_Matmul_with_diagonal_matrices_best_kernel.cu:43-62 (the 7 checks)
at::Tensor diag_mult(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.device().is_cuda(), "A must be a CUDA tensor");
    TORCH_CHECK(B.device().is_cuda(), "B must be a CUDA tensor");
    TORCH_CHECK(A.dim() == 1, "A must be 1-dimensional");
    TORCH_CHECK(B.dim() == 2, "B must be 2-dimensional");
    TORCH_CHECK(A.size(0) == B.size(0), "First dimension of B must match length of A");
    TORCH_CHECK(A.scalar_type() == at::kFloat, "A must be float32");
    TORCH_CHECK(B.scalar_type() == at::kFloat, "B must be float32");
    check_same_device(A, B);
    const int64_t N = A.size(0), M = B.size(1);
    at::Tensor a = A.contiguous(), Bc = B.contiguous();
    at::Tensor out = at::empty({N, M}, B.options());
    if (N == 0 || M == 0) return out;
    check_rc(mi_diag_mult_f32(a.data_ptr<float>(), Bc.data_ptr<float>(), out.data_ptr<float>(), N,
                              M, current_stream(B)),
             "diag_mult_cuda");
    return out;
}

// kernels/5_Matrix_scalar_multiplication_best_kernel.cu:47-71 (the 3 checks;
// output empty_like(A), no launch for an empty A)
at::Tensor matrix_scalar_mult(const at::Tensor& A, double s) {
    TORCH_CHECK(A.is_cuda(), "A must be a CUDA tensor");
    TORCH_CHECK(A.scalar_type() == at::kFloat, "A must be float32");
    TORCH_CHECK(A.is_contiguous(), "A must be contiguous");
    at::Tensor C = at::empty_like(A);
    if (A.numel() == 0) return C;
    check_rc(mi_matrix_scalar_mult_f32(A.data_ptr<float>(), C.data_ptr<float>(), A.numel(),
                                       static_cast<float>(s), current_stream(A)),
             "matrix_scalar_mult_cuda");
    return C;
}

// kernels/87_conv_pointwise_2D_best_kernel.cu:451-492.  The reference checks
// nothing and dispatches fp32/fp64/fp16/bf16; this operator is the fp32 path
// and rejects the rest, and checks the shapes the reference assumes (weight
// Cout x Cin [x 1 x 1], bias Cout).  Output: empty {N, Cout, H, W}.
at::Tensor pointwise_conv(const at::Tensor& input, const at::Tensor& weight,
                          const c10::optional<at::Tensor>& bias_opt) {
    TORCH_CHECK(input.dim() == 4, "input must be 4D (N, C_in, H, W)");
    TORCH_CHECK(weight.dim() == 2 || (weight.dim() == 4 && weight.size(2) == 1 && weight.size(3) == 1),
                "weight must be (C_out, C_in) or (C_out, C_in, 1, 1)");
    check_tensor(input, "input");
    check_tensor(weight, "weight");
    TORCH_CHECK(input.device() == weight.device(), "input and weight must be on the same device");
    const int64_t n = input.size(0), cin = input.size(1), h = input.size(2), w = input.size(3);
    const int64_t cout = weight.size(0);
    TORCH_CHECK(weight.size(1) == cin, "weight.size(1) must equal the input channels");
    at::Tensor bias;
    if (bias_opt.has_value() && bias_opt->defined()) {
        bias = *bias_opt;
        check_tensor(bias, "bias");
        TORCH_CHECK(bias.device() == input.device(), "bias must be on the input's device");
        TORCH_CHECK(bias.numel() == cout, "bias must have C_out elements");
        bias = bias.contiguous();
    }
    at::Tensor out = at::empty({n, cout, h, w}, input.options());
    if (out.numel() == 0) return out;
    at::Tensor x = input.contiguous(), wt = weight.contiguous();
    check_rc(mi_pointwise_conv_f32(x.data_ptr<float>(), wt.data_ptr<float>(),
                                   bias.defined() ? bias.data_ptr<float>() : nullptr,
                                   out.data_ptr<float>(), n, cin, cout, h * w, current_stream(input)),
             "pointwise_conv_cuda");
    return out;
}

// kernels/97_ScaledDotProductAttention_best_kernel.cu:256-296: Q, K, V are
// (batch, heads, seq, embed) fp16; the reference's three checks (:267-269)
// come first, then the ones its raw-pointer access assumes (shapes equal,
// fp16, CUDA).  Output empty_like(Q); workspace from the caching allocator.
at::Tensor fused_attention(const at::Tensor& Q, const at::Tensor& K, const at::Tensor& V) {
    TORCH_CHECK(Q.dim() == 4, "Q must be 4D (batch, heads, seq, embed)");
    const int64_t batch = Q.size(0), heads = Q.size(1), seq = Q.size(2), embed = Q.size(3);
    TORCH_CHECK(seq <= 512, "Sequence length exceeds MAX_SEQ_LENGTH.");
    TORCH_CHECK(embed == 1024, "Embedding dimension must be 1024.");
    TORCH_CHECK(embed % 32 == 0, "Embedding dimension must be divisible by warp size.");
    TORCH_CHECK(K.sizes() == Q.sizes() && V.sizes() == Q.sizes(), "Q, K and V must have the same shape");
    for (const at::Tensor* t : {&Q, &K, &V}) {
        TORCH_CHECK(t->is_cuda(), "Q, K and V must be CUDA tensors");
        TORCH_CHECK(t->scalar_type() == at::kHalf, "Q, K and V must be float16");
        TORCH_CHECK(t->device() == Q.device(), "Q, K and V must be on the same device");
    }
    at::Tensor out = at::empty_like(Q, at::MemoryFormat::Contiguous);
    if (out.numel() == 0) return out;
    at::Tensor q = Q.contiguous(), k = K.contiguous(), v = V.contiguous();
    const size_t ws_bytes = mi_sdpa_workspace_bytes(batch * heads, seq, embed);
    at::Tensor ws = at::empty({(int64_t)ws_bytes}, Q.options().dtype(at::kByte));
    check_rc(mi_sdpa_f16(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), batch * heads, seq,
                         embed, ws.data_ptr(), ws_bytes, current_stream(Q)),
             "fused_attention_cuda");
    return out;
}

// kernels/13_Matmul_for_symmetric_matrices_best_kernel.cu:134-151
at::Tensor symmetric_matmul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    const int64_t N = A.size(0);
    TORCH_CHECK(A.size(1) == N && B.size(0) == N && B.size(1) == N,
                "A and B must both be N x N with N = A.size(0)");
    check_pair(A, B);
    at::Tensor C = at::empty({N, N}, A.options());
    if (N == 0) return C;
    at::Tensor Ac = A.contiguous(), Bc = B.contiguous();
    const size_t wsb = mi_symmetric_matmul_workspace_bytes(N);
    at::Tensor ws = wsb ? at::empty({(int64_t)wsb}, A.options().dtype(at::kByte)) : at::Tensor();
    check_rc(mi_symmetric_matmul_f32(Ac.data_ptr<float>(), Bc.data_ptr<float>(),
                                     C.data_ptr<float>(), N, wsb ? ws.data_ptr() : nullptr, wsb,
                                     current_stream(A)),
             "symmetric_matmul_cuda");
    return C;
}

// kernels/14_Matmul_for_upper_triangular_matrices_best_kernel.cu:135-165 (5 checks)
at::Tensor upper_tri_matmul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(A.size(0) == A.size(1), "A must be square");
    TORCH_CHECK(B.size(0) == B.size(1), "B must be square");
    TORCH_CHECK(A.size(0) == B.size(0), "A and B must have the same size");
    check_pair(A, B);
    return gemm2d(A, false, B, false, MI_UPPER, "upper_tri_matmul_cuda");
}

// kernels/15_Matmul_for_lower_triangular_matrices_best_kernel.cu:155-206 (9 checks)
at::Tensor lower_tri_mul(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    const int64_t N = A.size(0);
    TORCH_CHECK(A.size(1) == N, "A must be square");
    TORCH_CHECK(B.size(0) == N, "B must have the same size as A");
    TORCH_CHECK(B.size(1) == N, "B must be square");
    TORCH_CHECK(A.is_cuda(), "A must be on CUDA");
    TORCH_CHECK(B.is_cuda(), "B must be on CUDA");
    check_pair(A, B);
    // the reference requires contiguous inputs (its last two checks); this
    // layer copies a non-contiguous input instead of rejecting it.
    return gemm2d(A.contiguous(), false, B.contiguous(), false, MI_LOWER, "lower_tri_mul_cuda");
}

// kernels/16_Matmul_with_transposed_A_best_kernel.cu:124-146
at::Tensor matmul_transposed_a(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(B.size(0) == A.size(0), "A and B must have the same number of rows");
    check_pair(A, B);
    return gemm2d(A, true, B, false, MI_DENSE, "matmul_transposed_cuda");
}

// kernels/17_Matmul_with_transposed_B_best_kernel.cu:267-286
at::Tensor matmul_transposed_b(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(A.size(1) == B.size(1), "A and B must have the same number of columns");
    check_pair(A, B);
    return gemm2d(A, false, B, true, MI_DENSE, "matmul_cuda");
}

// kernels/18_Matmul_with_transposed_both_best_kernel.cu:152-178
at::Tensor matmul_transposed_both(const at::Tensor& A, const at::Tensor& B) {
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    TORCH_CHECK(B.dim() == 2, "B must be 2D");
    TORCH_CHECK(A.size(0) == B.size(1), "A.size(0) must equal B.size(1)");
    check_pair(A, B);
    return gemm2d(A, true, B, true, MI_DENSE, "matmul_transposed_cuda");
}

}  // namespace mi355

// ---------------------------------------------------------------------------
// torch.ops.mi355.<op>: the same operators in the dispatcher, for graph use.
// CUDA (= HIP on ROCm) kernels are the functions above; Meta kernels give the
// output shape only (tracing, fake tensors).  There is deliberately no CPU
// kernel: a CPU tensor is an error, never a silent fallback.
// ---------------------------------------------------------------------------
namespace {

at::Tensor meta_like(const at::Tensor& t, at::IntArrayRef shape) { return at::empty(shape, t.options()); }

}  // namespace

TORCH_LIBRARY(mi355, m) {
    m.def("square_matmul(Tensor A, Tensor B) -> Tensor");            // PID 1
    m.def("matmul(Tensor A, Tensor B) -> Tensor");                   // PIDs 2, 8
    m.def("batched_matmul(Tensor A, Tensor B) -> Tensor");           // PID 3
    m.def("gemv(Tensor A, Tensor B) -> Tensor");                     // PID 4
    m.def("matrix_scalar_mult(Tensor A, float s) -> Tensor");        // PID 5
    m.def("matmul_large_k(Tensor A, Tensor B) -> Tensor");           // PID 6
    m.def("gemm_small_k(Tensor A, Tensor B) -> Tensor");             // PID 7
    m.def("tall_skinny_matmul(Tensor A, Tensor B) -> Tensor");       // PID 9
    m.def("tensor3d_matmul(Tensor A, Tensor B) -> Tensor");          // PID 10
    m.def("tensor4d_matmul(Tensor A, Tensor B) -> Tensor");          // PID 11
    m.def("diag_mult(Tensor A, Tensor B) -> Tensor");                // PID 12
    m.def("symmetric_matmul(Tensor A, Tensor B) -> Tensor");         // PID 13
    m.def("upper_tri_matmul(Tensor A, Tensor B) -> Tensor");         // PID 14
    m.def("lower_tri_mul(Tensor A, Tensor B) -> Tensor");            // PID 15
    m.def("matmul_transposed_a(Tensor A, Tensor B) -> Tensor");      // PID 16
    m.def("matmul_transposed_b(Tensor A, Tensor B) -> Tensor");      // PID 17
    m.def("matmul_transposed_both(Tensor A, Tensor B) -> Tensor");   // PID 18
    m.def("pointwise_conv(Tensor input, Tensor weight, Tensor? bias=None) -> Tensor");  // PID 87
    m.def("fused_attention(Tensor Q, Tensor K, Tensor V) -> Tensor");                   // PID 97
}

TORCH_LIBRARY_IMPL(mi355, CUDA, m) {
    m.impl("square_matmul", &mi355::square_matmul);
    m.impl("matmul", &mi355::matmul);
    m.impl("batched_matmul", &mi355::batched_matmul);
    m.impl("gemv", &mi355::gemv);
    m.impl("matrix_scalar_mult", &mi355::matrix_scalar_mult);
    m.impl("matmul_large_k", &mi355::matmul_large_k);
    m.impl("gemm_small_k", &mi355::gemm_small_k);
    m.impl("tall_skinny_matmul", &mi355::tall_skinny_matmul);
    m.impl("tensor3d_matmul", &mi355::tensor3d_matmul);
    m.impl("tensor4d_matmul", &mi355::tensor4d_matmul);
    m.impl("diag_mult", &mi355::diag_mult);
    m.impl("symmetric_matmul", &mi355::symmetric_matmul);
    m.impl("upper_tri_matmul", &mi355::upper_tri_matmul);
    m.impl("lower_tri_mul", &mi355::lower_tri_mul);
    m.impl("matmul_transposed_a", &mi355::matmul_transposed_a);
    m.impl("matmul_transposed_b", &mi355::matmul_transposed_b);
    m.impl("matmul_transposed_both", &mi355::matmul_transposed_both);
    m.impl("pointwise_conv", &mi355::pointwise_conv);
    m.impl("fused_attention", &mi355::fused_attention);
}

TORCH_LIBRARY_IMPL(mi355, Meta, m) {
    using T = const at::Tensor&;
    auto mm = [](T A, T B) { return meta_like(A, {A.size(0), B.size(1)}); };
    m.impl("square_matmul", mm);
    m.impl("matmul", mm);
    m.impl("matmul_large_k", mm);
    m.impl("gemm_small_k", mm);
    m.impl("tall_skinny_matmul", mm);
    m.impl("symmetric_matmul", mm);
    m.impl("upper_tri_matmul", mm);
    m.impl("lower_tri_mul", mm);
    m.impl("batched_matmul", [](T A, T B) { return meta_like(A, {A.size(0), A.size(1), B.size(2)}); });
    m.impl("gemv", [](T A, T B) { return meta_like(A, {A.size(0), 1}); });
    m.impl("matrix_scalar_mult", [](T A, double) { return at::empty_like(A); });
    m.impl("tensor3d_matmul", [](T A, T B) { return meta_like(A, {A.size(0), A.size(1), B.size(1)}); });
    m.impl("tensor4d_matmul",
           [](T A, T B) { return meta_like(A, {A.size(0), A.size(1), A.size(2), B.size(1)}); });
    m.impl("diag_mult", [](T A, T B) { return meta_like(B, {A.size(0), B.size(1)}); });
    m.impl("matmul_transposed_a", [](T A, T B) { return meta_like(A, {A.size(1), B.size(1)}); });
    m.impl("matmul_transposed_b", [](T A, T B) { return meta_like(A, {A.size(0), B.size(0)}); });
    m.impl("matmul_transposed_both", [](T A, T B) { return meta_like(A, {A.size(1), B.size(0)}); });
    m.impl("pointwise_conv", [](T x, T w, const c10::optional<at::Tensor>&) {
        return meta_like(x, {x.size(0), w.size(0), x.size(2), x.size(3)});
    });
    m.impl("fused_attention", [](T Q, T, T) { return at::empty_like(Q); });
}

// One Python submodule per reference file, exposing the reference's own
// function name (the names collide across files: matmul_cuda is PIDs 1, 2, 6,
// 8 and 17; matmul_transposed_cuda is 16 and 18; batched_matmul_cuda is 3 and 10).
PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "MI355X GEMM-family operators (drop-in for cuPilot-Kernels PIDs 1-18, 87 and 97)";
    struct Entry {
        const char* sub;
        const char* name;
        at::Tensor (*fn)(const at::Tensor&, const at::Tensor&);
    };
    const Entry entries[] = {
        {"p01", "matmul_cuda", &mi355::square_matmul},
        {"p02", "matmul_cuda", &mi355::matmul},
        {"p03", "batched_matmul_cuda", &mi355::batched_matmul},
        {"p04", "gemv_cuda", &mi355::gemv},
        {"p06", "matmul_cuda", &mi355::matmul_large_k},
        {"p07", "gemm_cuda", &mi355::gemm_small_k},
        {"p08", "matmul_cuda", &mi355::matmul},
        {"p09", "tall_skinny_matmul_cuda", &mi355::tall_skinny_matmul},
        {"p10", "batched_matmul_cuda", &mi355::tensor3d_matmul},
        {"p11", "tensor_matmul_cuda", &mi355::tensor4d_matmul},
        {"p12", "diag_mult_cuda", &mi355::diag_mult},
        {"p13", "symmetric_matmul_cuda", &mi355::symmetric_matmul},
        {"p14", "upper_tri_matmul_cuda", &mi355::upper_tri_matmul},
        {"p15", "lower_tri_mul_cuda", &mi355::lower_tri_mul},
        {"p16", "matmul_transposed_cuda", &mi355::matmul_transposed_a},
        {"p17", "matmul_cuda", &mi355::matmul_transposed_b},
        {"p18", "matmul_transposed_cuda", &mi355::matmul_transposed_both},
    };
    for (const Entry& e : entries) {
        auto sub = m.def_submodule(e.sub);
        sub.def(e.name, e.fn, pybind11::arg("A"), pybind11::arg("B"));
    }
    // PID 5 takes (Tensor A, float s); PID 87 (input, weight, optional bias)
    m.def_submodule("p05").def("matrix_scalar_mult_cuda", &mi355::matrix_scalar_mult,
                               pybind11::arg("A"), pybind11::arg("s"));
    m.def_submodule("p87").def("pointwise_conv_cuda", &mi355::pointwise_conv, pybind11::arg("input"),
                               pybind11::arg("weight"), pybind11::arg("bias_opt") = pybind11::none());
    // PID 97 takes (Q, K, V)
    m.def_submodule("p97").def("fused_attention_cuda", &mi355::fused_attention, pybind11::arg("Q"),
                               pybind11::arg("K"), pybind11::arg("V"));
    m.def("square_matmul", &mi355::square_matmul);
    m.def("matmul", &mi355::matmul);
    m.def("batched_matmul", &mi355::batched_matmul);
    m.def("gemv", &mi355::gemv);
    m.def("matmul_large_k", &mi355::matmul_large_k);
    m.def("gemm_small_k", &mi355::gemm_small_k);
    m.def("tall_skinny_matmul", &mi355::tall_skinny_matmul);
    m.def("tensor3d_matmul", &mi355::tensor3d_matmul);
    m.def("tensor4d_matmul", &mi355::tensor4d_matmul);
    m.def("diag_mult", &mi355::diag_mult);
    m.def("matrix_scalar_mult", &mi355::matrix_scalar_mult);
    m.def("pointwise_conv", &mi355::pointwise_conv);
    m.def("fused_attention", &mi355::fused_attention);
    m.def("symmetric_matmul", &mi355::symmetric_matmul);
    m.def("upper_tri_matmul", &mi355::upper_tri_matmul);
    m.def("lower_tri_mul", &mi355::lower_tri_mul);
    m.def("matmul_transposed_a", &mi355::matmul_transposed_a);
    m.def("matmul_transposed_b", &mi355::matmul_transposed_b);
    m.def("matmul_transposed_both", &mi355::matmul_transposed_both);
    m.def("version", []() { return std::string(mi_version()); });
}
