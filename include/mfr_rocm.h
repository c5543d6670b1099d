/*
 * mfr_rocm.h -- the C ABI of the MI355X (gfx950) backend for mensurflow's fp32 BLAS hot path.
 *
 * Everything the C++17 backend (mensurflow_amd/host/src/backends/rocm/) needs from HIP goes
 * through these functions; nothing above this header includes a HIP header. The library is
 * built by hipcc into libmfr_rocm.so.
 *
 * Conventions
 *   - Every function returns 0 on success and a nonzero MFR_E_* code on failure; the message of
 *     the last failure on the calling thread is returned by mfr_last_error(). No C++ exception
 *     crosses this boundary.
 *   - Sizes and strides are int64 element counts (not bytes). A "row stride" rs and "column
 *     stride" cs locate element (r, c) of a matrix at base + r*rs + c*cs.
 *   - Compute entry points enqueue work on a stream and return before the device finishes.
 *     mfr_memcpy_d2h and mfr_stream_sync wait for it.
 *   - Pointers passed to compute entry points are device pointers from mfr_malloc (or another
 *     HIP allocation on the stream's device).
 *
 * Each entry point names the interface of the reference (bakir004/mensurflow) it replaces.
 */
#ifndef MFR_ROCM_H
#define MFR_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MFR_OK = 0,
    MFR_E_INVALID = 1,     /* bad argument (the reference throws std::invalid_argument) */
    MFR_E_RUNTIME = 2,     /* HIP runtime failure (the reference throws std::runtime_error) */
    MFR_E_UNSUPPORTED = 3, /* a layout or size this build does not handle */
    MFR_E_NO_DEVICE = 4    /* no usable gfx950 device */
};

/* Activation applied in a GEMM epilogue or by mfr_bias_act.
 * GELU_TANH is mensurflow::gelu(x, approximate=true), GELU_ERF is gelu(x, false). */
enum { MFR_ACT_NONE = 0, MFR_ACT_GELU_TANH = 1, MFR_ACT_GELU_ERF = 2 };

/* Opaque stream: a HIP stream on one device plus the workspace its kernels use
 * (the reference keeps one Stream per device: src/backends/backend.hpp:32-44). */
typedef struct mfr_stream* mfr_stream_t;
typedef struct mfr_event* mfr_event_t;

/* ---- errors ------------------------------------------------------------------------------ */

/* Message of the last failure on this thread ("" if none). Replaces the reference's
 * runtime_error("CUDA <what> failed: ...") convention, src/backends/cuda/backend.cpp:22-34. */
const char* mfr_last_error(void);

/* ---- devices (Backend::device_count / Backend::info, src/backends/backend.hpp:51-60) ------ */

/* Number of usable gfx950 devices; 0 (and MFR_OK) when there is no driver or no device, so a
 * registry can drop the backend without an exception (src/core/registry.cpp:33-38). */
int mfr_get_device_count(int* count);

/* Device name (NUL-terminated, truncated to cap), total memory in bytes, compute units and the
 * peak engine clock in kHz. Any output pointer may be NULL. (DeviceInfo, backend.hpp:46-49) */
int mfr_get_device_info(int device, char* name, size_t cap, size_t* memory_bytes,
                        int* compute_units, int* clock_khz);

/* ---- memory (Backend::allocate / Buffer, src/backends/backend.hpp:16-30,62) --------------- */

/* bytes == 0 gives *ptr == NULL, as the reference's zero-byte Buffer has a null native(). */
int mfr_malloc(int device, size_t bytes, void** ptr);
/* NULL is accepted and ignored. */
int mfr_free(int device, void* ptr);

/* ---- streams (Stream, src/backends/backend.hpp:32-44) ------------------------------------- */

int mfr_stream_create(int device, mfr_stream_t* stream);
/* Wraps an existing hipStream_t (passed as void*) of `device`, e.g. a framework's current
 * stream; the HIP stream is not destroyed by mfr_stream_destroy. */
int mfr_stream_wrap(int device, void* hip_stream, mfr_stream_t* stream);
int mfr_stream_destroy(mfr_stream_t stream);
/* Blocks until all work queued on the stream has finished (Stream::synchronize). */
int mfr_stream_sync(mfr_stream_t stream);
/* The underlying hipStream_t (as void*), for interop and profiling. */
void* mfr_stream_handle(mfr_stream_t stream);
int mfr_stream_device(mfr_stream_t stream);

/* Host -> device; complete on return, so src may be reused (Stream::copy_h2d). Copies of 1 MiB
 * or more from pageable memory go through the stream's two 16 MiB pinned staging slots (allocated
 * on first use, freed with the stream), the CPU's copy into one overlapping the DMA of the other;
 * mfr_memcpy_d2h likewise. Calls on one stream from several threads take turns. */
int mfr_memcpy_h2d(mfr_stream_t stream, void* dst, const void* src, size_t bytes);
/* Device -> host; waits for all earlier work on the stream (Stream::copy_d2h). */
int mfr_memcpy_d2h(mfr_stream_t stream, void* dst, const void* src, size_t bytes);
/* Device -> device, ordered on the stream; returns before it finishes. */
int mfr_memcpy_d2d(mfr_stream_t stream, void* dst, const void* src, size_t bytes);

/* ---- events (device-side timing; the reference times with host clocks, benchmarks/bench.hpp) */

int mfr_event_create(mfr_event_t* event);
int mfr_event_destroy(mfr_event_t event);
int mfr_event_record(mfr_event_t event, mfr_stream_t stream);
/* Milliseconds between two recorded events; waits for `end`. */
int mfr_event_elapsed_ms(mfr_event_t start, mfr_event_t end, float* ms);

/* ---- GEMM -------------------------------------------------------------------------------- */

#define MFR_MAX_BATCH_DIMS 4

/* One (batched) GEMM with a fused epilogue:
 *
 *   C[b](i,j) = act( fl( fl( fl(alpha * sum_p A[b](i,p) * B[b](p,j)) + fl(beta * C0[b](i,j)) )
 *                        + bias[j] ) )
 *
 * for every batch index b of a batch shape of up to MFR_MAX_BATCH_DIMS dimensions (outermost
 * first); matrix b of an operand starts at base + sum_d b_d * batch_stride_d, and a batch
 * stride of 0 repeats one matrix (a broadcast batch dimension). A is op(A) [m, k] and B is
 * op(B) [k, n], each given by its own row and column strides, so a transposed operand is a
 * swapped stride pair. The fl() steps are the reference's separate roundings: matmul, then
 * mul by alpha, scal by beta and add (src/ops/blas.cpp:234-262), or the batched GEMM's finish
 * pass (src/backends/cpu/ops/gemm/gemm_batched.cpp:12-28); the bias step is bias_add
 * (src/backends/cpu/ops/elementwise/elementwise.cpp:128-137) and act is gelu
 * (elementwise.cpp:173-194). alpha == 1 skips the multiply, c0 == NULL or beta == 0 skips the
 * C0 term, bias == NULL skips the bias.
 *
 * Each operand needs a unit stride in one of its two matrix dimensions (row-major or
 * transposed); C has column stride 1. c0 may equal c (in place). k == 0 gives the epilogue of
 * a zero product. The products are summed in fp32 on the fp32 matrix cores
 * (v_mfma_f32_32x32x2_f32), in a different order from the CPU's packed kernel.
 *
 * Replaces: the Matmul kernel (src/backends/cpu/backend.cpp:131-164), the GemmBatched kernel
 * (backend.cpp:239-291), and the 4-dispatch composition of mensurflow::gemm
 * (src/ops/blas.cpp:234-262) when called as one fused op.
 */
typedef struct mfr_gemm_desc {
    int64_t m, n, k;
    int32_t batch_dims;                       /* 0 .. MFR_MAX_BATCH_DIMS */
    int32_t act;                              /* MFR_ACT_* */
    int64_t batch[MFR_MAX_BATCH_DIMS];        /* batch sizes, outermost first */
    const float* a;
    int64_t a_rs, a_cs;
    int64_t a_bs[MFR_MAX_BATCH_DIMS];
    const float* b;
    int64_t b_rs, b_cs;
    int64_t b_bs[MFR_MAX_BATCH_DIMS];
    float* c;
    int64_t c_rs;
    int64_t c_bs[MFR_MAX_BATCH_DIMS];
    const float* c0;                          /* may be NULL; may equal c */
    int64_t c0_rs;
    int64_t c0_bs[MFR_MAX_BATCH_DIMS];
    const float* bias;                        /* [n] or NULL; shared by every batch */
    float alpha, beta;
    int32_t tile;                             /* MFR_TILE_AUTO or a fixed MFR_TILE_* */
    int32_t stage;                            /* MFR_STAGE_* */
    int32_t splits;                           /* 0 = AUTO, or 1 .. MFR_MAX_SPLITS depth ranges */
    int32_t flags;                            /* 0 or MFR_GEMM_CAUSAL */
} mfr_gemm_desc;

/* mfr_gemm_desc.flags. MFR_GEMM_CAUSAL: in every batch matrix, C(i, j) = -inf wherever j > i (the
 * top-left causal mask of attention's scores, as where(keep, scores, -inf) with keep(i, j) =
 * j <= i writes them: src/ops/attention.cpp:85-96), and those outputs are not computed; the rest
 * as without the flag. Only the panel path takes it (MFR_TILE_PANEL, or AUTO where the panel
 * path fits); anything else is MFR_E_UNSUPPORTED. */
enum { MFR_GEMM_CAUSAL = 1 };

/* Operand staging of mfr_sgemm. The fast loads read 4 floats at once, which needs an operand's
 * unit-stride extent and its other strides to be multiples of 4 and its base 16-byte aligned
 * (X[4093,1023] row-major is not). Such an operand can first be copied, zero-padded to that
 * shape, into the stream's workspace (one extra pass over it). AUTO stages when the product is
 * large (>= 2^30 flops) and the copy is small next to it (<= 1 byte per 64 flops), except that
 * under the 256x256 tile it stages only operands with a unit stride along the depth and reads the
 * others in place; the result is the same either way. Without staging, the 256x256 tile reads
 * such operands in place, with 4-byte buffer loads that write LDS directly. */
enum { MFR_STAGE_AUTO = 0, MFR_STAGE_NEVER = 1, MFR_STAGE_ALWAYS = 2 };

/* Workgroup tile of mfr_sgemm (rows x cols x depth slice). AUTO picks one from the shape (with
 * the split count): a time model of the busiest CU's tiles (ceil(tiles / CUs) of them, each its
 * area x (depth + a fixed per-tile overhead) at the tile's measured rate, slower when a SIMD holds
 * fewer than 3 wavefronts), and the high-occupancy tiles for a depth <= 128. A fixed tile is what
 * a tuner sets (the reference's TuningConfig,
 * src/core/dispatcher.hpp:145-149). Every tile gives the same results up to summation order. */
enum {
    MFR_TILE_AUTO = 0,
    MFR_TILE_256x256 = 1, /* 16 wavefronts of 64x64, 1 workgroup per CU */
    MFR_TILE_128x128 = 2, /* 4 wavefronts of 64x64, 2 per CU */
    MFR_TILE_128x64 = 3,  /* 4 wavefronts of 64x32, depth slice 16, up to 5 per CU */
    MFR_TILE_64x128 = 4,  /* 4 wavefronts of 32x64, depth slice 16 */
    MFR_TILE_64x64 = 5,   /* 4 wavefronts of 32x32, 4 per CU */
    MFR_TILE_THIN = 6,    /* no MFMA: at most 8 output columns (or rows) as dot products */
    MFR_TILE_PANEL = 7,   /* k <= 64: 8 wavefronts keep 256 rows of A, stream B and C past them */
    MFR_TILE_COUNT = 8
};

/* The thin path (MFR_TILE_THIN) streams the long operand once and keeps the other, at most 8
 * columns wide, in LDS: for n <= 8 with A read along k (unit stride along K), or m <= 8 with B
 * read along k. Elsewhere a fixed THIN fails with MFR_E_UNSUPPORTED; it runs no split. AUTO
 * prices it against the MFMA tiles. */

/* The panel path (MFR_TILE_PANEL) is for a short depth and a large output, such as attention's
 * scores q k^T: a workgroup holds 256 rows of A in registers for the whole launch and walks the
 * columns of C, 64 at a time, with the matching rows of B copied into LDS and C written while
 * the next columns are multiplied, so the stores overlap the MFMA work instead of following it.
 * It takes 1 <= k <= 64 with both operands read along k (unit stride along K) by 16-byte loads
 * (their k, other strides and bases 16-byte aligned), no activation and no split; alpha, beta *
 * C0 and a bias as everywhere. The sums are the MFMA tiles' own, so the results are the same bit
 * for bit. Elsewhere a fixed PANEL fails with MFR_E_UNSUPPORTED. AUTO takes it where it fits for
 * outputs of more than 128 rows and at least 2^22 elements. */

/* Split-K of mfr_sgemm. A product with few output tiles and a long depth (256 x 256 x 16384)
 * would leave most compute units idle, so its depth may be cut into `splits` ranges (each a
 * multiple of 32 deep; fewer ranges than asked when the depth is short): each range's raw sums go
 * to the stream's workspace (splits * m * n * batch floats), and a second pass adds the ranges in
 * order and applies the epilogue with the same roundings. AUTO picks the tile and the count
 * together from a time model (no split when the output fills the device, ranges >= 256 deep,
 * partial sums <= 1 GiB) and falls back to no split when the workspace cannot be had; a fixed
 * count fails with MFR_E_RUNTIME then. Results are deterministic; the summation order, hence
 * the rounding, depends on the count. */
#define MFR_MAX_SPLITS 64

int mfr_sgemm(mfr_stream_t stream, const mfr_gemm_desc* desc);

/* mfr_sgemm without any device allocation. No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It makes the same plan as mfr_sgemm and gives the same bits, but puts the split-K
 * partial sums and staged operands in a fixed scratch array of MFR_SGEMM_SCRATCH_BYTES per device
 * (a static device array, resident until the process ends) instead of the stream's workspace. A
 * plan that needs more (the split-K sums are splits*m*n*batch floats, a staged operand its
 * zero-padded copy) takes the fallbacks mfr_sgemm takes when its workspace cannot be had, where
 * the descriptor leaves them to AUTO (automatic splits become one range, automatic staging reads
 * the operands in place: the same results up to summation order); what still needs more fails
 * with MFR_E_INVALID before anything is launched. Products with aligned operands and no split
 * need none. Every call on one device shares that device's array, so calls
 * that overlap on one device (on two streams, or from two threads) race; the array keeps the last
 * call's contents, and nothing in it needs to start at zero. The first call on a device looks up
 * the array's address there. */
#define MFR_SGEMM_SCRATCH_BYTES ((size_t)64 << 20)
int mfr_sgemm_noalloc(mfr_stream_t stream, const mfr_gemm_desc* desc);

/* Edge peeling (tile and splits both AUTO): a dimension a few rows past a multiple of a big tile
 * (N = 4099 = 16 x 256 + 3) would cost that tile a whole extra wave of tiles for a sliver of work,
 * so such a remainder (at most a quarter of the tile) may run as a separate launch with its own
 * tile and split count, when the time model prices that at least 5% lower. Up to 4 launches: the main
 * rectangle, the right strip, the bottom strip, the corner. */

/* What mfr_sgemm would run for desc on device `device`, without launching anything: the tile
 * (an MFR_TILE_* other than AUTO; AUTO when there is nothing to compute), whether operands
 * are staged (MFR_STAGE_ALWAYS) or read in place (MFR_STAGE_NEVER), and the depth ranges
 * (1 = no split; 0 when there is nothing to compute), each of the main region, and the number of
 * output regions launched separately (1, or 2-4 with edge peeling; 0 when there is nothing to
 * compute). Validates desc as mfr_sgemm
 * does and fails with the same status where mfr_sgemm would (MFR_E_UNSUPPORTED for a fixed
 * 256x256 tile with staging off and operands 16-byte loads cannot read). For tuners: the default
 * a search starts from, and whether a (tile, stage) point can run (the reference's
 * TunableKernel::defaults / allowed, src/core/dispatcher.hpp:226-239). */
int mfr_sgemm_plan(int device, const mfr_gemm_desc* desc, int32_t* tile, int32_t* stage,
                   int32_t* splits, int32_t* regions);

/* Plain row-major convenience form: C[m,n] = alpha*op(A)*op(B) + beta*C0 with leading
 * dimensions lda/ldb/ldc (BLAS-style trans flags, row-major storage). c0 may be NULL. */
int mfr_sgemm_rm(mfr_stream_t stream, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
                 float alpha, const float* a, int64_t lda, const float* b, int64_t ldb, float beta,
                 const float* c0, float* c, int64_t ldc);

/* ---- GEMV / matvec ------------------------------------------------------------------------- */

/* y = alpha * op(A) * x + beta * y0, A row-major [rows, cols] with row stride lda >= cols,
 * op(A) = A (trans == 0, y has `rows` entries) or A^T (trans != 0, y has `cols` entries).
 * y0 may be NULL only when beta == 0; beta != 0 without y0 is MFR_E_INVALID, the reference's
 * "gemv: beta requires an output vector" (src/ops/blas.cpp:155-157). Accumulates in double and
 * rounds once, as
 * mensurflow::cpu::gemv_f32 (src/backends/cpu/ops/blas/blas.cpp:66-79):
 *   y[i] = (float)( (double)alpha * sum + (double)(float)(beta * y0[i]) ).
 * Deterministic: the same inputs give the same bits on every call (fixed reduction order, no
 * float atomics). Replaces the Gemv kernel (src/backends/cpu/backend.cpp:121-126). */
int mfr_sgemv(mfr_stream_t stream, int trans, int64_t rows, int64_t cols, float alpha,
              const float* a, int64_t lda, const float* x, float beta, const float* y0, float* y);

/* y[m] = A[m,k] * x[k], double accumulation (mensurflow::cpu::matvec_f32, blas.cpp:55-64).
 * Replaces the Matvec kernel (src/backends/cpu/backend.cpp:115-119). */
int mfr_smatvec(mfr_stream_t stream, int64_t m, int64_t k, const float* a, int64_t lda,
                const float* x, float* y);

/* *out = sum over i < n of x[i] * y[i] (unit strides; out is one float of device memory, 0 for
 * n = 0): each product in double (exact), the sum in double in a fixed order that depends on n
 * alone, rounded once, as the reference's dot_f32 (src/backends/cpu/ops/blas/blas.cpp:14-21)
 * adds them in double. Replaces the Dot kernel that mensurflow::dot dispatches
 * (src/ops/blas.cpp:41-68), which the CUDA backend serves with cublasSdot
 * (src/backends/cuda/backend.cpp:131-133). */
int mfr_sdot(mfr_stream_t stream, int64_t n, const float* x, const float* y, float* out);

/* ---- elementwise, softmax, argmax ---------------------------------------------------------- */

/* y[r, j] = act(x[r, j] + bias[j]) over a contiguous [rows, cols] matrix; bias may be NULL
 * (then y = act(x), the Gelu kernel). act = MFR_ACT_NONE with a bias is bias_add.
 * Replaces BiasAdd (src/backends/cpu/backend.cpp:762-767, elementwise.cpp:128-137) and Gelu
 * (backend.cpp:658-661, elementwise.cpp:173-194). x may equal y. */
int mfr_bias_act(mfr_stream_t stream, const float* x, const float* bias, float* y, int64_t rows,
                 int64_t cols, int act);

/* out[i] = cond[i] ? x[i] : y[i] over n contiguous elements (cond is 1 byte per element).
 * Replaces Where (src/backends/cpu/backend.cpp:625-630, elementwise.cpp:64-70). */
int mfr_where(mfr_stream_t stream, const uint8_t* cond, const float* x, const float* y, float* out,
              int64_t n);

/* out = cond ? x : y over an ndim-dimensional output `shape` (out contiguous, row-major), each
 * operand read through its own element strides, 0 on a broadcast dimension (ndim <= 8, strides
 * >= 0). The form of Where for operands that broadcast: attention's -inf scalar and its [Lq, Lk]
 * mask expanded over [B, H, Lq, Lk] are read once each instead of packed to the scores' shape,
 * which is what the reference does (src/ops/elementwise.cpp:454-481). Same selection as
 * mfr_where (elementwise.cpp:64-70). */
int mfr_where_nd(mfr_stream_t stream, int32_t ndim, const int64_t* shape, const uint8_t* cond,
                 const int64_t* cond_strides, const float* x, const int64_t* x_strides,
                 const float* y, const int64_t* y_strides, float* out);

/* Softmax of x viewed as [outer, length, inner] along the middle axis (contiguous).
 * Float maximum (a NaN poisons the line), float exp(x - max), double sum, one float scale;
 * a line whose maximum is -inf (every element masked) gives zeros.
 * Replaces Softmax (src/backends/cpu/backend.cpp:549-553, softmax/softmax.cpp:13-49). */
int mfr_softmax(mfr_stream_t stream, const float* x, float* y, int64_t outer, int64_t length,
                int64_t inner);

/* out[r] = index of the first maximum of row r of a contiguous [rows, width] matrix; the first
 * NaN wins. Replaces Argmax (src/backends/cpu/backend.cpp:799-803, reduction.cpp:284-296). */
int mfr_argmax(mfr_stream_t stream, const float* x, int64_t* out, int64_t rows, int64_t width);

/* out[i] = a[i] + b[i] (op MFR_EW_ADD), a[i] - b[i] (MFR_EW_SUB), a[i] * b[i] (MFR_EW_MUL), or
 * alpha * a[i] (MFR_EW_SCAL, b unused) over n contiguous elements, one fp32 rounding each.
 * Replaces the Add, Sub, Mul and Scal kernels (registered at src/backends/cpu/backend.cpp:856-867;
 * add_f32/sub_f32/mul_f32 at src/backends/cpu/ops/elementwise/elementwise.cpp:72-91, scal_f32 at
 * ops/blas/blas.cpp:23-28) that mensurflow::gemm's unfused composition dispatches
 * (src/ops/blas.cpp:246-257); Add, Sub and Mul are also the ops the CUDA backend registers
 * (src/backends/cuda/backend.cpp:231-235). */
enum { MFR_EW_ADD = 0, MFR_EW_MUL = 1, MFR_EW_SCAL = 2, MFR_EW_SUB = 3 };
int mfr_elementwise(mfr_stream_t stream, int op, const float* a, const float* b, float alpha,
                    float* out, int64_t n);

/* ---- fused attention ---------------------------------------------------------------------- */

/* Scaled dot-product attention in one kernel, without materialising the [.., lq, lk] scores:
 *
 *   out[b](i, :) = sum_j p_ij v[b](j, :),  p_ij = softmax_j(s_ij),
 *   s_ij = fl(scale * q[b](i, :) . k[b](j, :)), or -inf where the mask is 0, where causal and
 *   j > i (top-left aligned), or where j >= lk.
 *
 * The softmax is the online (running-maximum) form: each block of keys rescales the partial
 * sums by exp(m_old - m_new), and the output is divided by the row's sum once at the end; a row
 * with every key removed gives zeros, a NaN score gives a NaN row. q [.., lq, d], k [.., lk, d],
 * v [.., lk, d] and out [.., lq, d] have unit stride along d, row strides and batch strides
 * (0 = broadcast) that are multiples of 4 floats and 16-byte aligned bases; d is a multiple of 16,
 * at most 128.
 * Anything else is MFR_E_UNSUPPORTED (the caller composes the op instead). The mask (NULL, or
 * 1 byte per element: nonzero keeps) has any strides, 0 for broadcast dimensions. scale 0 means
 * fl(1/sqrt(d)).
 *
 * Replaces: mensurflow::attention's composition (src/ops/attention.cpp:48-98) -- a batched GEMM
 * for the scores, where() with -inf for masked and causal positions, softmax over the keys
 * (src/backends/cpu/ops/softmax/softmax.cpp:13-49) and a batched GEMM with v -- as one op. It
 * sums in a different order and normalises after the weighted sum, so it agrees with the
 * composition to fp32 rounding (max relative error 1e-5*sqrt(lk) of sum_j |p_ij v_jc|), not
 * bit for bit. */
typedef struct mfr_attention_desc {
    int64_t lq, lk, d;
    int32_t batch_dims;                       /* 0 .. MFR_MAX_BATCH_DIMS */
    int32_t causal;
    int64_t batch[MFR_MAX_BATCH_DIMS];
    const float* q;
    int64_t q_rs, q_bs[MFR_MAX_BATCH_DIMS];
    const float* k;
    int64_t k_rs, k_bs[MFR_MAX_BATCH_DIMS];
    const float* v;
    int64_t v_rs, v_bs[MFR_MAX_BATCH_DIMS];
    float* out;
    int64_t out_rs, out_bs[MFR_MAX_BATCH_DIMS];
    const uint8_t* mask;                      /* may be NULL */
    int64_t mask_rs, mask_cs, mask_bs[MFR_MAX_BATCH_DIMS];
    float scale;
    int32_t reserved;
} mfr_attention_desc;

int mfr_attention(mfr_stream_t stream, const mfr_attention_desc* desc);

/* ---- layout ------------------------------------------------------------------------------- */

#define MFR_MAX_COPY_DIMS 8

/* Packs a strided view (shape/strides in elements, up to MFR_MAX_COPY_DIMS dimensions, stride 0
 * allowed) into contiguous row-major dst, element size 1, 2, 4 or 8 bytes. The device-side
 * form of Tensor::contiguous(), which the reference stages through host memory for non-CPU
 * devices (src/core/tensor.cpp:208-230). */
int mfr_strided_copy(mfr_stream_t stream, const void* src, void* dst, int32_t elem_size,
                     int32_t ndim, const int64_t* shape, const int64_t* strides);

/* Fills n elements of elem_size bytes (1, 2, 4 or 8) with the bit pattern `value`
 * (the low elem_size bytes are used). */
int mfr_fill(mfr_stream_t stream, void* dst, int32_t elem_size, int64_t n, uint64_t value);

#ifdef __cplusplus
}
#endif

#endif /* MFR_ROCM_H */
