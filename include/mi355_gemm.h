/*
 * mi355_gemm.h -- C ABI of the MI355X (gfx950) GEMM-family library
 * (libmi355gemm.so).
 *
 * Drop-in boundary for the GEMM-family operators of champloo2878/cuPilot-Kernels
 * (kernels/1..4, 6..18).  Each reference operator is a libtorch host function
 * `torch::Tensor <name>(torch::Tensor A, torch::Tensor B)`; the entry points
 * below are what a C FFI for those operators binds: device pointers, sizes and
 * a stream, no torch types.  Each one cites the reference function it replaces.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers to fp32 data; matrices are row-major with
 *     the stated leading dimension (elements).
 *   - `stream` is a hipStream_t passed as void*; NULL is the null stream.
 *     Work is enqueued asynchronously; nothing synchronises the host.
 *   - The library never allocates or frees device memory and keeps no pointer
 *     after returning.  Entry points that need scratch take a workspace; its
 *     size comes from the matching *_workspace_bytes query.  (The one
 *     exception, mi_gemm_f32_noalloc, keeps its scratch in a fixed array the
 *     library holds on each device.)
 *   - Return value: MI_OK (0); a negative mi_status for an invalid argument
 *     (checked before any launch); a positive hipError_t for a launch failure.
 *     mi_status_string() turns either into text.
 *   - A zero-size dimension is valid: the output is written with zeros where it
 *     has elements (or left untouched if it has none) and no MFMA kernel runs.
 *   - Reentrant: no global mutable state; concurrent calls on different
 *     streams are independent.
 */
#ifndef MI355_GEMM_H
#define MI355_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef MI_API
#define MI_API __attribute__((visibility("default")))
#endif

typedef enum {
    MI_OK = 0,
    MI_ERR_NULL_POINTER = -1,
    MI_ERR_BAD_SIZE = -2,       /* negative size, or size beyond int32 tiles */
    MI_ERR_BAD_LAYOUT = -3,     /* op / structure enum out of range */
    MI_ERR_BAD_LD = -4,         /* leading dimension smaller than the row */
    MI_ERR_NOT_SQUARE = -5,     /* structured op on a non-square problem */
    MI_ERR_WORKSPACE = -6,      /* workspace missing or too small */
    MI_ERR_NO_DEVICE = -7,      /* no HIP device / device query failed */
    MI_ERR_ALIGNMENT = -8,      /* a pointer is not 16-byte aligned where required */
    MI_ERR_SCRATCH_LIMIT = -9   /* mi_gemm_f32_noalloc: a plan_override forces a plan
                                   needing more scratch than MI_NOALLOC_SCRATCH_BYTES */
} mi_status;

typedef enum { MI_OP_N = 0, MI_OP_T = 1 } mi_op;

typedef enum {
    MI_DENSE = 0,
    MI_LOWER = 1,   /* C = tril(tril(A) . tril(B)), exact zeros above the diagonal */
    MI_UPPER = 2,   /* C = triu(triu(A) . triu(B)), exact zeros below the diagonal
                       (both: while the call runs, C's zero triangle may hold
                       partial sums and a work counter; it is +0.0 when the
                       stream reaches the next operation) */
    MI_SYMMETRIC = 3 /* C = op_a(A) . op_b(B) for square operands (the reference's
                        symmetric operator): planned and computed exactly as the
                        dense product, so a non-symmetric input gets its own
                        product, as in kernels/13_...:134-151 */
} mi_structure;

/*
 * Generic strided-batched contraction C[b] = op_a(A[b]) . op_b(B[b]).
 *   op_a = N: A[b] is M x K with row stride lda;  T: A[b] is stored K x M (lda).
 *   op_b = N: B[b] is K x N with row stride ldb;  T: B[b] is stored N x K (ldb).
 *   C[b] is M x N with row stride ldc.  stride_* are batch strides in elements
 *   (stride_b = 0 broadcasts one B to every batch).
 * Every named entry point below is a thin front of this one.
 */
typedef struct {
    const float* A;
    const float* B;
    float* C;
    int64_t M, N, K, batch;
    int64_t lda, ldb, ldc;
    int64_t stride_a, stride_b, stride_c;
    int32_t op_a, op_b;       /* mi_op */
    int32_t structure;        /* mi_structure; square, batch 1, N/N layouts */
    int32_t plan_override;    /* 0 = scheduler's choice; else (tests, tuning) bits 0-3 tile
                                 config id (mi_plan.plan_id), bit 4 stream-K where it applies,
                                 bit 5 never stream-K, bit 6 (MI_PLAN_NO_PACK) never pack the
                                 operands, bit 7 (MI_PLAN_PACK) pack them where packing applies
                                 (the other bits then apply to the packed product), bits 8-19
                                 split count, bits 20-29 raster group rows, bit 30
                                 (MI_PLAN_SK_RANGES) stream-K over contiguous K-slice ranges
                                 instead of phases (mi_plan.sk_phases); a config the problem
                                 cannot take is ignored */
    void* workspace;
    size_t workspace_bytes;
    const float* bias_m;      /* NULL, or M floats: C[b][i][j] = (sum over k) + bias_m[i],
                                 one fp32 add after the full sum, the same for every
                                 batch; dense structure and op_a = op_b = N only */
} mi_gemm_args;

/* plan_override bits 6 and 7 (operand packing, see mi_plan.packed) */
#define MI_PLAN_NO_PACK 0x40
#define MI_PLAN_PACK 0x80
/* plan_override bit 30 (see mi_plan.sk_phases) */
#define MI_PLAN_SK_RANGES 0x40000000

/* Scheduler decision for one contraction (host-only, no device access). */
typedef struct {
    int32_t plan_id;        /* kernel instantiation */
    int32_t block_m, block_n, block_k;
    int32_t tiles_m, tiles_n;
    int32_t split_k;        /* 1 = no split; else K is cut into split_k chunks */
    int64_t k_chunk;        /* elements of K per split (multiple of block_k) */
    int32_t group_m;        /* tile rows per raster group */
    int64_t num_tiles;      /* output tiles per (split, batch) */
    int64_t grid;           /* workgroups launched per (split, batch); each walks tiles
                               wg, wg + grid, ... (persistent; stream-K plans: see
                               mi_gemm_work_item) */
    size_t workspace_bytes; /* split-K partial tiles, or stream-K partial tiles (one
                               slot per workgroup) */
    int32_t stream_k;       /* 1: stream-K schedule -- the last sk_tiles tiles' K-slices
                               are dealt out evenly over the grid workgroups (the
                               first num_tiles - sk_tiles tiles stay whole), partial
                               tiles are added in by a fixed-order fixup pass */
    int64_t sk_tiles;
    int32_t packed;         /* 1: A and B are first packed into the workspace
                               K-contiguous with K zero-padded to packed_k, and the
                               fields above describe the N/T product of the packed
                               operands; workspace_bytes includes the packed copies */
    int64_t packed_k;
    int32_t sk_phases;      /* stream-K plans: 0 -- each workgroup reduces one contiguous
                               range of the tiles' K-slices (each starting at its own
                               offset); > 0 -- that many phases, in each of which a run of
                               workgroups reduces the same K range of neighbouring tiles,
                               starting together, so that one XCD's workgroups read the
                               same slices (mi_gemm_work_item shows the segments) */
} mi_plan;

/* One work item of a workgroup under a plan (host introspection). */
typedef struct {
    int32_t tile_m, tile_n; /* output tile */
    int64_t k_begin, k_end; /* K range it reduces */
    int32_t dest;           /* 0: written to C (a whole tile, or the k = 0 head of a
                               stream-K tile); 1: written to workspace slot `slot`
                               (a split-K split, or a stream-K partial tile) */
    int32_t slot;
} mi_work_item;

MI_API int mi_gemm_f32(const mi_gemm_args* args, void* stream);
MI_API size_t mi_gemm_workspace_bytes(const mi_gemm_args* args);
/* Allocation-free variant of mi_gemm_f32 (no counterpart in the reference; for
 * callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * result as mi_gemm_f32 -- the same plan, kernels and reduction order as a
 * call given a workspace of mi_gemm_workspace_bytes(args) bytes, so the same
 * bits -- but args->workspace and args->workspace_bytes are ignored: the
 * scratch (split-K and stream-K partial tiles, packed operand copies) goes to
 * a fixed MI_NOALLOC_SCRATCH_BYTES array the library holds on each device
 * (for the life of the process) instead.
 *   - A problem whose preferred plan needs more scratch than that is planned
 *     as mi_gemm_f32 plans it with a workspace of MI_NOALLOC_SCRATCH_BYTES
 *     bytes (fewer splits, or no packed copies; an unsplit plan needing no
 *     scratch always exists), so its result may then differ from
 *     mi_gemm_f32's with the preferred workspace in the last bits.
 *   - Only a plan_override that forces a plan needing more scratch than that
 *     returns MI_ERR_SCRATCH_LIMIT, before anything is launched.
 *   - The first call on a device looks up that device's copy of the array
 *     (hipGetSymbolAddress, once per device); make that first call outside
 *     graph capture.  Calls, and captures, after it allocate nothing.
 *   - Every call on one device shares its array: calls that overlap on one
 *     device (unordered streams or host threads) race.  Nothing in the array
 *     needs clearing between calls. */
#define MI_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
MI_API int mi_gemm_f32_noalloc(const mi_gemm_args* args, void* stream);
/* Pure host function: what mi_gemm_f32 would launch on a device with num_cus
 * compute units.  Exposed for tests and tuning. */
MI_API int mi_gemm_plan(const mi_gemm_args* args, int32_t num_cus, mi_plan* out);

/* Scheduler introspection (no reference counterpart; for tests and tuning):
 * the output tile (tile_m, tile_n) and K range [k_begin, k_end) of work item
 * `item` (0 <= item < mi_plan.num_tiles; workgroup w runs items w, w + grid,
 * ...) of split `split` under the plan mi_gemm_f32 would use on a device with
 * num_cus compute units.  Returns 1 for a compute tile, 0 for a
 * structural-zero tile (triangular products), 2 for a K chunk of a long
 * triangular tile whose partial sum is parked in the mirror tile
 * (tile_n, tile_m) of the zero triangle and added in by a finishing pass
 * (the chunked work list of triangular products with N % 256 == 0; its items
 * run longest first, claimed in list order by persistent workgroups as they
 * free up, so which workgroup runs an item is decided at run time), 3 for a
 * zero-triangle tile that list's workgroups write with +0.0 once its compute
 * items are claimed (items num_tiles, num_tiles + 1, ...: every zero tile
 * that parks no partial, except the one holding the item counter; the
 * finishing pass writes the rest), a negative mi_status on error. */
MI_API int mi_gemm_tile_of(const mi_gemm_args* args, int32_t num_cus, int64_t item, int32_t split,
                           int32_t* tile_m, int32_t* tile_n, int64_t* k_begin, int64_t* k_end);

/* Scheduler introspection for dense persistent plans, stream-K included (no
 * reference counterpart; for tests and tuning): work item `item` (0, 1, ...
 * in the order it runs) of workgroup wg (0 <= wg < mi_plan.grid) of split
 * `split`.  Returns 1 and fills *out, 0 when the workgroup has no such item,
 * MI_ERR_BAD_LAYOUT for triangular and A-panel plans (mi_gemm_tile_of covers
 * those), another negative mi_status on error. */
MI_API int mi_gemm_work_item(const mi_gemm_args* args, int32_t num_cus, int64_t wg, int32_t split,
                             int64_t item, mi_work_item* out);

/* Stream-K fixup (no reference counterpart; for tests and tuning): stream-K
 * tile t (0 <= t < mi_plan.sk_tiles) is output tile (tile_m, tile_n); the
 * fixup pass adds workspace slots first_slot, first_slot + 1, ...,
 * first_slot + n_slots - 1 into it, in that order (n_slots = 0: one
 * workgroup reduced the whole tile).  A slot whose workgroup got no K-slices
 * holds nothing and is skipped.  Returns 1, or a negative mi_status (also for
 * a plan that is not stream-K). */
MI_API int mi_gemm_sk_fixup_of(const mi_gemm_args* args, int32_t num_cus, int64_t t,
                               int32_t* tile_m, int32_t* tile_n, int64_t* first_slot,
                               int64_t* n_slots);

/* ---- one entry point per reference operator ------------------------------ */

/* Workspace of the dense product entry points (those taking `workspace,
 * workspace_bytes`): device memory, 256-byte aligned, of the size their
 * *_workspace_bytes query returns for the same extents -- then the call runs
 * the plan mi_gemm_f32 runs with the workspace mi_gemm_workspace_bytes asks
 * for (split-K, stream-K, packed operand copies; the same bits as the
 * operator layer).  A smaller workspace (NULL with 0 bytes included) restricts
 * the scheduler to the plans that fit it, down to those needing none, and the
 * result may then differ in the last bits.  The query is 0 when no plan of the
 * problem wants one. */

/* kernels/1_Square_matrix_multiplication_best_kernel.cu:189 matmul_cuda(A, B):
 * C = A . B, all N x N. */
MI_API size_t mi_square_matmul_workspace_bytes(int64_t N);
MI_API int mi_square_matmul_f32(const float* A, const float* B, float* C, int64_t N,
                                void* workspace, size_t workspace_bytes, void* stream);

/* kernels/2_Standard_matrix_multiplication_best_kernel.cu:117 matmul_cuda and
 * kernels/8_Matmul_with_irregular_shapes_best_kernel.cu:155 matmul_cuda:
 * C (M x N) = A (M x K) . B (K x N), any sizes. */
MI_API size_t mi_matmul_workspace_bytes(int64_t M, int64_t K, int64_t N);
MI_API int mi_matmul_f32(const float* A, const float* B, float* C,
                  int64_t M, int64_t K, int64_t N,
                  void* workspace, size_t workspace_bytes, void* stream);

/* kernels/3_Batched_matrix_multiplication_best_kernel.cu:113 batched_matmul_cuda:
 * C[b] (M x N) = A[b] (M x K) . B[b] (K x N). */
MI_API size_t mi_batched_matmul_workspace_bytes(int64_t batch, int64_t M, int64_t K, int64_t N);
MI_API int mi_batched_matmul_f32(const float* A, const float* B, float* C,
                          int64_t batch, int64_t M, int64_t K, int64_t N,
                          void* workspace, size_t workspace_bytes, void* stream);

/* kernels/4_Matrix_vector_multiplication_best_kernel.cu:84 gemv_cuda:
 * y (M) = A (M x K) . x (K).  Uses a workspace of mi_gemv_workspace_bytes(M, K)
 * bytes for its deterministic split-K partial sums (may be 0 bytes). */
MI_API size_t mi_gemv_workspace_bytes(int64_t M, int64_t K);
MI_API int mi_gemv_f32(const float* A, const float* x, float* y, int64_t M, int64_t K,
                void* workspace, size_t workspace_bytes, void* stream);

/* kernels/6_Matmul_with_large_K_dimension_best_kernel.cu:128 matmul_cuda:
 * C (M x N) = A (M x K) . B (K x N) for K >> M, N; single-launch split-K with a
 * fixed-order reduction (bitwise deterministic).  Workspace from
 * mi_matmul_large_k_workspace_bytes. */
MI_API size_t mi_matmul_large_k_workspace_bytes(int64_t M, int64_t K, int64_t N);
MI_API int mi_matmul_large_k_f32(const float* A, const float* B, float* C,
                          int64_t M, int64_t K, int64_t N,
                          void* workspace, size_t workspace_bytes, void* stream);

/* kernels/7_Matmul_with_small_K_dimension_best_kernel.cu:80 gemm_cuda:
 * C (M x N) = A (M x K) . B (K x N) for small K (store-bound). */
MI_API int mi_gemm_small_k_f32(const float* A, const float* B, float* C,
                        int64_t M, int64_t K, int64_t N, void* stream);

/* kernels/9_Tall_skinny_matrix_multiplication_best_kernel.cu:145
 * tall_skinny_matmul_cuda: A is M x N, B is N x M, C (M x M) = A . B. */
MI_API int mi_tall_skinny_matmul_f32(const float* A, const float* B, float* C,
                              int64_t M, int64_t N, void* stream);

/* kernels/10_3D_tensor_matrix_multiplication_best_kernel.cu:180 batched_matmul_cuda:
 * out[n] (M x L) = A[n] (M x K) . B (K x L), A is N x M x K. */
MI_API size_t mi_tensor3d_matmul_workspace_bytes(int64_t N, int64_t M, int64_t K, int64_t L);
MI_API int mi_tensor3d_matmul_f32(const float* A, const float* B, float* out,
                           int64_t N, int64_t M, int64_t K, int64_t L,
                           void* workspace, size_t workspace_bytes, void* stream);

/* kernels/11_4D_tensor_matrix_multiplication_best_kernel.cu:132 tensor_matmul_cuda:
 * out[b,i,j,:] = A[b,i,j,:] . B, A is b x i x j x l, B is l x k. */
MI_API size_t mi_tensor4d_matmul_workspace_bytes(int64_t b, int64_t i, int64_t j, int64_t l,
                                                 int64_t k);
MI_API int mi_tensor4d_matmul_f32(const float* A, const float* B, float* out,
                           int64_t b, int64_t i, int64_t j, int64_t l, int64_t k,
                           void* workspace, size_t workspace_bytes, void* stream);

/* kernels/12_Matmul_with_diagonal_matrices_best_kernel.cu:43 diag_mult_cuda:
 * out (N x M) = diag(a) . B, a has length N; one fp32 multiply per element. */
MI_API int mi_diag_mult_f32(const float* a, const float* B, float* out,
                     int64_t N, int64_t M, void* stream);

/* kernels/5_Matrix_scalar_multiplication_best_kernel.cu:47 matrix_scalar_mult_cuda:
 * C[i] = A[i] * s for the n floats of a contiguous array; one fp32 multiply
 * per element. */
MI_API int mi_matrix_scalar_mult_f32(const float* A, float* C, int64_t n, float s,
                              void* stream);

/* kernels/87_conv_pointwise_2D_best_kernel.cu:451 pointwise_conv_cuda (a 1x1
 * convolution; the reference computes it at :174-446):
 *   output[n][o][p] = sum_c weight[o][c] * input[n][c][p] + bias[o]
 * with input N x Cin x HW, weight Cout x Cin (a Cout x Cin x 1 x 1 tensor),
 * output N x Cout x HW, all contiguous, bias NULL or Cout floats (added once,
 * after the full sum).  One batched contraction, the weight broadcast over
 * the images. */
MI_API int mi_pointwise_conv_f32(const float* input, const float* weight, const float* bias,
                          float* output, int64_t batch, int64_t in_channels,
                          int64_t out_channels, int64_t hw, void* stream);

/* kernels/97_ScaledDotProductAttention_best_kernel.cu:256 fused_attention_cuda
 * (reference kernel :136-250): for each of batch_heads (batch x heads) heads,
 *   O = softmax(Q . K^T / sqrt(embed)) . V
 * with Q, K, V, O contiguous fp16 (IEEE binary16) arrays of batch_heads x seq
 * x embed, fp32 arithmetic inside, one rounding to fp16 at the end.  embed
 * must be a multiple of 64 and the four pointers 16-byte aligned.  The
 * workspace (device memory, mi_sdpa_workspace_bytes) holds the attention
 * weights of up to 128 heads at a time, and for seq > 512 their fp32 scores. */
MI_API size_t mi_sdpa_workspace_bytes(int64_t batch_heads, int64_t seq, int64_t embed);
MI_API int mi_sdpa_f16(const void* Q, const void* K, const void* V, void* O, int64_t batch_heads,
                int64_t seq, int64_t embed, void* workspace, size_t workspace_bytes,
                void* stream);

/* kernels/13_Matmul_for_symmetric_matrices_best_kernel.cu:134
 * symmetric_matmul_cuda: C = A . B for N x N A and B (meant for symmetric
 * inputs; like the reference kernel, :57 and :134-151, it relies on no
 * symmetry and returns A . B for any input). */
MI_API size_t mi_symmetric_matmul_workspace_bytes(int64_t N);
MI_API int mi_symmetric_matmul_f32(const float* A, const float* B, float* C, int64_t N,
                            void* workspace, size_t workspace_bytes, void* stream);

/* kernels/14_Matmul_for_upper_triangular_matrices_best_kernel.cu:135
 * upper_tri_matmul_cuda: C = triu(triu(A) . triu(B)), N x N; zero tiles are
 * skipped and the lower triangle is written with exact zeros. */
MI_API int mi_upper_tri_matmul_f32(const float* A, const float* B, float* C, int64_t N,
                            void* stream);

/* kernels/15_Matmul_for_lower_triangular_matrices_best_kernel.cu:155
 * lower_tri_mul_cuda: C = tril(tril(A) . tril(B)), N x N. */
MI_API int mi_lower_tri_mul_f32(const float* A, const float* B, float* C, int64_t N,
                         void* stream);

/* kernels/16_Matmul_with_transposed_A_best_kernel.cu:124 matmul_transposed_cuda:
 * C (M x N) = A^T . B with A stored K x M and B K x N. */
MI_API size_t mi_matmul_transposed_a_workspace_bytes(int64_t M, int64_t K, int64_t N);
MI_API int mi_matmul_transposed_a_f32(const float* A, const float* B, float* C,
                               int64_t M, int64_t K, int64_t N,
                               void* workspace, size_t workspace_bytes, void* stream);

/* kernels/17_Matmul_with_transposed_B_best_kernel.cu:267 matmul_cuda:
 * C (M x N) = A . B^T with A M x K and B stored N x K. */
MI_API size_t mi_matmul_transposed_b_workspace_bytes(int64_t M, int64_t K, int64_t N);
MI_API int mi_matmul_transposed_b_f32(const float* A, const float* B, float* C,
                               int64_t M, int64_t K, int64_t N,
                               void* workspace, size_t workspace_bytes, void* stream);

/* kernels/18_Matmul_with_transposed_both_best_kernel.cu:152 matmul_transposed_cuda:
 * C (M x N) = A^T . B^T with A stored K x M and B stored N x K. */
MI_API size_t mi_matmul_transposed_both_workspace_bytes(int64_t M, int64_t K, int64_t N);
MI_API int mi_matmul_transposed_both_f32(const float* A, const float* B, float* C,
                                  int64_t M, int64_t K, int64_t N,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* ---- utilities ------------------------------------------------------------ */

/* Counter-based input generator (no reference counterpart; test and benchmark
 * inputs): out[i] = float(splitmix64((seed << 40) + offset + i) >> 40) * 2^-23 - 1,
 * uniform on [-1, 1), bit-identical to the host generator. */
MI_API int mi_fill_uniform_f32(float* out, int64_t n, uint64_t seed, int64_t offset, void* stream);

MI_API const char* mi_status_string(int status);
/* Library version, e.g. "mi355_gemm 0.1.0 gfx950". */
MI_API const char* mi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MI355_GEMM_H */
