// Device code of the fp32 MFMA GEMM: the tile kernel and its operand loader. Included by
// gemm.hip (the C ABI entry points and tile selection). See gemm.hip for the design.
#pragma once

#include "common.hpp"

#include <type_traits>

namespace mfr::gemm {

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Word 3 of a raw buffer resource on gfx9 (32-bit dword format, no swizzle): the buffer unit
// checks each access against the resource's size in bytes, returning zeros for loads past it and
// dropping stores past it.
constexpr int kBufferWord3 = 0x00020000;

struct GemmParams {
    const float* a;
    const float* b;
    float* c;
    const float* c0;
    const float* bias;
    int64_t m, n, k;
    int64_t a_rs, a_cs, b_rs, b_cs, c_rs, c0_rs;
    int64_t batch[MFR_MAX_BATCH_DIMS];
    int64_t a_bs[MFR_MAX_BATCH_DIMS], b_bs[MFR_MAX_BATCH_DIMS];
    int64_t c_bs[MFR_MAX_BATCH_DIMS], c0_bs[MFR_MAX_BATCH_DIMS];
    int32_t batch_dims;
    int32_t act;
    int64_t batch_count;
    int32_t tiles_m, tiles_n;
    int32_t group_m;
    float alpha, beta;
    // Split-K: the depth is cut into `splits` ranges of k_per_split (a multiple of the depth
    // slice; the last may be shorter). With splits > 1 each workgroup writes its raw fp32 sums to
    // partial[split][batch][m][n] (dense, batch in linear order) instead of running the
    // epilogue; split_reduce_kernel then adds the splits and applies it.
    int64_t k_per_split;
    int32_t splits;
    float* partial;
    // Nonzero: C is written with non-temporal (streaming) stores on interior tiles without C0 or
    // an activation. Set for outputs larger than the last-level cache whose rows all start on
    // 128-byte lines (partial lines would be merged in L2 otherwise).
    int32_t stream_c;
    // Nonzero: C(i, j) = -inf for j > i in every batch matrix (MFR_GEMM_CAUSAL; panel path only).
    int32_t causal;
};

// Global -> register -> LDS copy of one operand slice: ROWS rows (M for A, N for B) by KT depth.
// KMAJ: unit stride along the depth (element (r, p) at base + r*row_stride + p).
// otherwise: unit stride along the rows (element (r, p) at base + p*k_stride + r).
// V: 4 = 16-byte loads along the unit-stride dimension (its extent and the other stride are
// multiples of 4, the base 16-byte aligned), 1 = 4-byte loads.
template <int ROWS, int KT, bool KMAJ, int V, int THREADS> struct SliceLoader {
    static constexpr int kUnits = ROWS * KT / V;        // loads per slice
    static constexpr int kPerThread = kUnits / THREADS;
    static_assert(kUnits % THREADS == 0, "slice must split evenly over the workgroup");
    // LDS row pitch: [ROWS][KT+4] (K-major) or [KT][ROWS+8].
    static constexpr int kPitch = KMAJ ? KT + 4 : ROWS + 8;
    static constexpr int kFloats = KMAJ ? ROWS * (KT + 4) : KT * (ROWS + 8);

    using Vec = typename std::conditional<V == 4, float4, float>::type;
    Vec reg[kPerThread];

    // (row, depth) of this thread's i-th load, in elements.
    __device__ __forceinline__ static void coords(int i, int& r, int& p) {
        const int u = static_cast<int>(threadIdx.x) + i * THREADS;
        if constexpr (KMAJ) {
            constexpr int per_row = KT / V;
            r = u / per_row;
            p = (u % per_row) * V;
        } else {
            constexpr int per_depth = ROWS / V;
            p = u / per_depth;
            r = (u % per_depth) * V;
        }
    }

    // base points at element (row 0, depth k0) of the slice. rows_left / k_left: how many rows
    // and depths of the slice are inside the matrix (>= ROWS / KT for an interior slice).
    __device__ __forceinline__ void load(const float* base, int64_t row_stride, int64_t k_stride,
                                         int rows_left, int k_left) {
        const bool full = rows_left >= ROWS && k_left >= KT;
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            int r, p;
            coords(i, r, p);
            const float* src = KMAJ ? base + r * row_stride + p : base + p * k_stride + r;
            if (full || (r < rows_left && p < k_left)) {
                if constexpr (V == 4) {
                    reg[i] = *reinterpret_cast<const float4*>(src);
                } else {
                    reg[i] = *src;
                }
            } else {
                if constexpr (V == 4) {
                    reg[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    reg[i] = 0.f;
                }
            }
        }
    }

    __device__ __forceinline__ void store(float* lds) const {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            int r, p;
            coords(i, r, p);
            float* dst = KMAJ ? lds + r * kPitch + p : lds + p * kPitch + r;
            if constexpr (V == 4) {
                *reinterpret_cast<float4*>(dst) = reg[i];
            } else {
                *dst = reg[i];
            }
        }
    }

    // The four MFMA-step values of fragment row `row` (0..ROWS-1) for depth group g (8 depths):
    // lanes 0-31 (half 0) take depths 8g+0..3, lanes 32-63 (half 1) depths 8g+4..7.
    __device__ __forceinline__ static void fragment(const float* lds, int row, int g, int half,
                                                    float out[4]) {
        if constexpr (KMAJ) {
            const float4 v = *reinterpret_cast<const float4*>(lds + row * kPitch + 8 * g + 4 * half);
            out[0] = v.x;
            out[1] = v.y;
            out[2] = v.z;
            out[3] = v.w;
        } else {
            // One per-lane address; the depth offsets are constants the LDS reads carry as
            // immediates (per-depth addresses would each take a register across the depth loop).
            const float* column = lds + 4 * half * kPitch + row;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                out[s] = column[(8 * g + s) * kPitch];
            }
        }
    }
};

// Writes a wavefront's accumulators: block (i, j), element e is C(row0 + 32i + 8(e/4) + e%4,
// col0 + 32j), as
//   C = act(fl(fl(fl(alpha * acc) + fl(beta * C0)) + bias))      (RAW: C = acc),
// the C0 term only when c0 is non-null, so the roundings are the reference's. Without a bias, -0
// is added (x + -0 is x for every x, -0 included), which spares a test per element. alpha * acc
// is exact for alpha == 1. INTERIOR: every row and column is
// inside C (no checks). C0 == kC0Batched: c0 is non-null and a row-block's C0 values are all
// loaded before any is used, so the loads overlap; kC0None: no C0; kC0Checked: c0 checked per
// element (one copy of the code for both cases). STREAM: non-temporal stores.
enum { kC0None = 0, kC0Batched = 1, kC0Checked = 2 };
// ROWS_PAST_M: a tile whose columns are all inside C and whose rows may run past m; every element
// is computed and stored through a buffer resource of m rows, which drops the stores to rows past
// m (no per-element test; the caller checks that (m + 256) * c_rs * 4 fits 32 bits).
// JS: the column step between accumulator blocks: 32 (block j holds columns col0 + 32 j ..), or
// 1 for the paired layout of sgemm_pair_kernel (a lane's block j holds column col0 + j, col0 even).
template <int FM, int FN, int ACT, bool INTERIOR, bool RAW, int C0, bool STREAM = false,
          bool ROWS_PAST_M = false, int JS = 32>
__device__ __forceinline__ void write_tile(const floatx16 (&acc)[FM][FN], float* c, int64_t c_rs,
                                           const float* c0, int64_t c0_rs, const GemmParams& p,
                                           int64_t row0, int64_t col0,
                                           const double* exp_table = nullptr) {
    static_assert(!ROWS_PAST_M || (!INTERIOR && C0 == kC0None && !STREAM), "row-edge copy");
    // Byte offsets into C within the resource (32 bits by the caller's check).
    // The record count is a 32-bit unsigned field; the caller keeps 4 (m + 256) c_rs below 2^32.
    const __amdgpu_buffer_rsrc_t c_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        c, 0, ROWS_PAST_M ? static_cast<int>(static_cast<uint32_t>(4 * p.m * c_rs)) : 0,
        kBufferWord3);
    // Kernel parameters read once: per element, the compiler would reload them after each store.
    const float alpha = p.alpha;
    const float beta = p.beta;
    const float* const bias_base = RAW ? nullptr : p.bias;
    // The bias of each column block, loaded before any store and waited for at once (the empty
    // asm reads it): a first use inside a predicated element would leave the load pending on the
    // paths that skip it, and every later element would wait for the memory counter, which also
    // counts the stores issued since.
    float bias_of[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t col = col0 + JS * j;
        bias_of[j] = bias_base != nullptr && (INTERIOR || col < p.n) ? bias_base[col] : -0.0f;
        asm volatile("" ::"v"(bias_of[j]));
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int64_t row_i = row0 + 32 * i;
        float* c_i = c + row_i * c_rs + col0;
        float c0v[FN][16];
        if constexpr (C0 == kC0Batched) {
            const float* c0_i = c0 + row_i * c0_rs + col0;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int dr = 8 * (e / 4) + e % 4;
                    const bool inside = INTERIOR || (col0 + JS * j < p.n && row_i + dr < p.m);
                    c0v[j][e] = inside ? c0_i[dr * c0_rs + JS * j] : 0.0f;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t col = col0 + JS * j;
            if (!INTERIOR && !ROWS_PAST_M && col >= p.n) {
                continue;
            }
            const float bias = bias_of[j];
            // Elements outside C (rows past m) are computed all the same and only the loads and
            // stores are predicated, so no branch separates them.
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int dr = 8 * (e / 4) + e % 4;
                const bool row_ok = INTERIOR || ROWS_PAST_M || row_i + dr < p.m;
                float v = acc[i][j][e];
                if constexpr (!RAW) {
                    v = alpha * v;
                    if constexpr (C0 == kC0Batched) {
                        const float scaled = beta * c0v[j][e];
                        v = v + scaled;
                    } else if constexpr (C0 == kC0Checked) {
                        if (c0 != nullptr) {
                            const float c0_value = row_ok ? c0[(row_i + dr) * c0_rs + col] : 0.0f;
                            const float scaled = beta * c0_value;
                            v = v + scaled;
                        }
                    }
                    v = v + bias; // -0 without a bias: x + -0 is x
                    if constexpr (ACT == MFR_ACT_GELU_TANH) {
                        v = gelu_math::gelu_tanh(v, exp_table);
                    } else if constexpr (ACT != MFR_ACT_NONE) {
                        v = mfr::dev::gelu(v, ACT);
                    }
                }
                if constexpr (ROWS_PAST_M) {
                    const uint32_t offset =
                        static_cast<uint32_t>(4 * ((row_i + dr) * c_rs + col0 + JS * j));
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), c_rsrc,
                                                          offset, 0, 0);
                } else if (row_ok) {
                    if constexpr (STREAM) {
                        __builtin_nontemporal_store(v, &c_i[dr * c_rs + JS * j]);
                    } else {
                        c_i[dr * c_rs + JS * j] = v;
                    }
                }
            }
        }
    }
}

// The epilogue for activation ACT. Without one it is dispatched on C0 and on whether the tile is
// interior. The tanh gelu has three copies without C0 (the MLP's case): interior tiles, tiles
// whose rows alone run past m (stores through a buffer resource that drops those rows), and other
// edges. With C0 tested and loaded between the elements, each element would wait for the memory
// counter, which also counts the stores before it. Every other gelu epilogue is one checked copy.
template <int FM, int FN, int ACT, int JS = 32>
__device__ __forceinline__ void epilogue(const floatx16 (&acc)[FM][FN], float* c, int64_t c_rs,
                                         const float* c0, int64_t c0_rs, const GemmParams& p,
                                         int64_t row0, int64_t col0, bool interior,
                                         bool rows_only_edge, const double* exp_table) {
    if constexpr (ACT == MFR_ACT_GELU_TANH) {
        if (interior && c0 == nullptr) {
            write_tile<FM, FN, ACT, true, false, kC0None, false, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0, col0,
                                                          exp_table);
        } else if (rows_only_edge && c0 == nullptr) {
            write_tile<FM, FN, ACT, false, false, kC0None, false, true, JS>(acc, c, c_rs, c0, c0_rs, p,
                                                                        row0, col0, exp_table);
        } else if (c0 == nullptr) {
            write_tile<FM, FN, ACT, false, false, kC0None, false, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0, col0,
                                                           exp_table);
        } else {
            write_tile<FM, FN, ACT, false, false, kC0Checked, false, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                              col0, exp_table);
        }
    } else if constexpr (ACT != MFR_ACT_NONE) {
        write_tile<FM, FN, ACT, false, false, kC0Checked, false, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0, col0);
    } else if (c0 != nullptr) {
        if (interior) {
            write_tile<FM, FN, ACT, true, false, kC0Batched, false, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                             col0);
        } else {
            write_tile<FM, FN, ACT, false, false, kC0Batched, false, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                              col0);
        }
    } else {
        if (interior && p.stream_c) {
            write_tile<FM, FN, ACT, true, false, kC0None, true, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                                col0);
        } else if (interior) {
            write_tile<FM, FN, ACT, true, false, kC0None, false, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0, col0);
        } else {
            write_tile<FM, FN, ACT, false, false, kC0None, false, false, JS>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                           col0);
        }
    }
}

// Which output tile a workgroup computes: the XCD-aware remap of the hardware workgroup index,
// grouped row-major order within the batch, the depth split outermost; and the operand offsets
// of its batch entry.
struct TileWork {
    int64_t split, batch_linear, m0, n0;
    int64_t off_a, off_b, off_c, off_c0;
    int rows_a, rows_b; // rows of A (M) and of B (N) inside the matrix, capped at the tile
    int64_t k_begin, kk; // depth range [k_begin, k_begin + kk)
};

template <int BM, int BN> __device__ __forceinline__ TileWork tile_work(const GemmParams& p) {
    TileWork w;
    // Every index here is below the launch's workgroup count, which the host keeps under 2^31,
    // so the decomposition runs in 32-bit unsigned arithmetic: a 64-bit division is a long
    // scalar instruction sequence, and every wavefront of every workgroup runs these (about a
    // thousand instructions before a small tile's first load in 64 bits).
    const uint32_t tiles_m = static_cast<uint32_t>(p.tiles_m);
    const uint32_t tiles_n = static_cast<uint32_t>(p.tiles_n);
    const uint32_t tiles_per_batch = tiles_m * tiles_n;
    const uint32_t tiles_per_split = tiles_per_batch * static_cast<uint32_t>(p.batch_count);
    const uint32_t total = tiles_per_split * static_cast<uint32_t>(p.splits);
    const uint32_t hw = blockIdx.x;
    const uint32_t per_xcd = total / 8;
    const uint32_t logical_all = hw < per_xcd * 8 ? (hw % 8) * per_xcd + hw / 8 : hw;
    const uint32_t split = logical_all / tiles_per_split;
    const uint32_t logical = logical_all - split * tiles_per_split;
    const uint32_t batch_linear = logical / tiles_per_batch;
    const uint32_t t = logical - batch_linear * tiles_per_batch;
    // Groups of group_m tile-rows; a group taller than the matrix is the matrix (the same order,
    // and group_tiles stays within the batch's tile count).
    const uint32_t gm = static_cast<uint32_t>(p.group_m) < tiles_m
                            ? static_cast<uint32_t>(p.group_m)
                            : tiles_m;
    const uint32_t group_tiles = gm * tiles_n;
    const uint32_t group = t / group_tiles;
    const uint32_t first_m = group * gm;
    const uint32_t rows_in_group = tiles_m - first_m < gm ? tiles_m - first_m : gm;
    const uint32_t in_group = t - group * group_tiles;
    const int64_t tile_m = first_m + in_group % rows_in_group;
    const int64_t tile_n = in_group / rows_in_group;
    w.split = split;
    w.batch_linear = batch_linear;
    uint32_t batch_index = batch_linear;
    w.off_a = w.off_b = w.off_c = w.off_c0 = 0;
    for (int d = p.batch_dims - 1; d >= 0; --d) {
        const uint32_t extent = static_cast<uint32_t>(p.batch[d]);
        const int64_t idx = batch_index % extent;
        batch_index /= extent;
        w.off_a += idx * p.a_bs[d];
        w.off_b += idx * p.b_bs[d];
        w.off_c += idx * p.c_bs[d];
        w.off_c0 += idx * p.c0_bs[d];
    }
    w.m0 = tile_m * BM;
    w.n0 = tile_n * BN;
    w.rows_a = p.m - w.m0 < BM ? static_cast<int>(p.m - w.m0) : BM;
    w.rows_b = p.n - w.n0 < BN ? static_cast<int>(p.n - w.n0) : BN;
    w.k_begin = w.split * p.k_per_split;
    w.kk = p.k - w.k_begin < p.k_per_split ? p.k - w.k_begin : p.k_per_split;
    return w;
}

// One depth slice of MFMAs from the LDS tiles sa, sb: the wavefront's FM x FN 32x32 blocks over
// the 8-deep groups it takes (wave_k, wave_k + WAVES_K, ...).
template <typename LoadA, typename LoadB, int KT, int FM, int FN, int WM, int WN, int WAVES_K>
__device__ __forceinline__ void slice_mfma(floatx16 (&acc)[FM][FN], const float* sa,
                                           const float* sb, int wave_m, int wave_n, int wave_k,
                                           int half, int r32) {
#pragma unroll
    for (int gi = 0; gi < KT / 8 / WAVES_K; ++gi) {
        const int g = gi * WAVES_K + wave_k;
        float fa[FM][4];
        float fb[FN][4];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            LoadA::fragment(sa, wave_m * WM + i * 32 + r32, g, half, fa[i]);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            LoadB::fragment(sb, wave_n * WN + j * 32 + r32, g, half, fb[j]);
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][st], fb[j][st],
                                                                      acc[i][j], 0, 0, 0);
                }
            }
        }
    }
}

// The end of a tile: split-K partial sums, or the epilogue with the activation chosen once.
template <int BM, int BN, int WM, int WN, int FM, int FN, int JS = 32>
__device__ __forceinline__ void finish_tile(const floatx16 (&acc)[FM][FN], const GemmParams& p,
                                            const TileWork& w, int wave_m, int wave_n, int half,
                                            int r32, const double* exp_table) {
    // Accumulator e of block (i, j) is C(row, col) with row = 32i + 8(e/4) + 4*half + e%4,
    // col = 32j + lane%32 (v_mfma_f32_32x32x2_f32 layout), or 2 (lane%32) + j when paired.
    const int64_t row0 = w.m0 + wave_m * WM + 4 * half;
    const int64_t col0 = w.n0 + wave_n * WN + (JS == 32 ? r32 : 2 * r32);
    const bool interior = w.m0 + BM <= p.m && w.n0 + BN <= p.n;
    // Rows past m only, and C's byte offsets (rows past m included) within 32 bits.
    const bool rows_only_edge = !interior && w.n0 + BN <= p.n &&
                                (p.m + BM) * p.c_rs * 4 < (int64_t{1} << 32);
    if (p.partial != nullptr) {
        // Split-K: raw sums only, to partial[split][batch] (dense m x n).
        float* part = p.partial + (w.split * p.batch_count + w.batch_linear) * p.m * p.n;
        if (interior) {
            write_tile<FM, FN, MFR_ACT_NONE, true, true, kC0None, false, false, JS>(
                acc, part, p.n, nullptr, 0, p, row0, col0);
        } else {
            write_tile<FM, FN, MFR_ACT_NONE, false, true, kC0None, false, false, JS>(
                acc, part, p.n, nullptr, 0, p, row0, col0);
        }
        return;
    }
    float* c_base = p.c + w.off_c;
    const float* c0_base = p.c0 != nullptr && p.beta != 0.0f ? p.c0 + w.off_c0 : nullptr;
    // One activation per branch (uniform), so each epilogue is straight-line code: unrolled
    // over every accumulator, the three would not fit the instruction cache together.
    if (p.act == MFR_ACT_NONE) {
        epilogue<FM, FN, MFR_ACT_NONE, JS>(acc, c_base, p.c_rs, c0_base, p.c0_rs, p, row0, col0,
                                       interior, rows_only_edge, exp_table);
    } else if (p.act == MFR_ACT_GELU_TANH) {
        epilogue<FM, FN, MFR_ACT_GELU_TANH, JS>(acc, c_base, p.c_rs, c0_base, p.c0_rs, p, row0, col0,
                                            interior, rows_only_edge, exp_table);
    } else {
        epilogue<FM, FN, MFR_ACT_GELU_ERF, JS>(acc, c_base, p.c_rs, c0_base, p.c0_rs, p, row0, col0,
                                           interior, rows_only_edge, exp_table);
    }
}

// WAVES_K > 1: WAVES_K sets of WAVES_M x WAVES_N wavefronts share each depth slice, set w taking
// its 8-deep groups w, w + WAVES_K, ...; the sets' accumulators are then added through LDS, in
// set order, and set 0 runs the epilogue. It gives a small grid (a workgroup per CU) several
// wavefronts per SIMD without splitting the depth across workgroups.
template <int BM, int BN, int KT, int WAVES_M, int WAVES_N, bool AK, bool BK, int VA, int VB,
          int WAVES_K = 1>
__global__ __launch_bounds__(WAVES_M * WAVES_N * WAVES_K * 64) void sgemm_kernel(GemmParams p) {
    constexpr int THREADS = WAVES_M * WAVES_N * WAVES_K * 64;
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int FM = WM / 32; // 32x32 accumulator blocks per wavefront, along M
    constexpr int FN = WN / 32;
    static_assert(KT % 8 == 0 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
    static_assert((KT / 8) % WAVES_K == 0, "each wavefront set takes whole 8-deep groups");
    using LoadA = SliceLoader<BM, KT, AK, VA, THREADS>;
    using LoadB = SliceLoader<BN, KT, BK, VB, THREADS>;
    __shared__ float smem[2 * (LoadA::kFloats + LoadB::kFloats)];
    // Buffer `which` (0 or 1) of each operand's double-buffered slice.
    auto lds_a = [&](int which) { return smem + which * LoadA::kFloats; };
    auto lds_b = [&](int which) { return smem + 2 * LoadA::kFloats + which * LoadB::kFloats; };

    const TileWork w = tile_work<BM, BN>(p);
    const float* a_base = p.a + w.off_a + w.m0 * p.a_rs + w.k_begin * p.a_cs;
    const float* b_base = p.b + w.off_b + w.n0 * p.b_cs + w.k_begin * p.b_rs;
    // Per slice the bases advance by KT depths.
    const int64_t a_step = KT * p.a_cs;
    const int64_t b_step = KT * p.b_rs;

    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    // With one set, the set index is the constant 0, which keeps every fragment's LDS offset
    // a compile-time constant (a run-time 0 cost 3 % at 3000^3 on the 64x64 tile).
    const int wave_mn = WAVES_K == 1 ? wave : wave % (WAVES_M * WAVES_N);
    const int wave_k =
        WAVES_K == 1 ? 0 : __builtin_amdgcn_readfirstlane(wave / (WAVES_M * WAVES_N));
    const int wave_m = wave_mn / WAVES_N;
    const int wave_n = wave_mn % WAVES_N;
    const int half = lane / 32;
    const int r32 = lane % 32;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                acc[i][j][e] = 0.0f;
            }
        }
    }

    const int64_t kk = w.kk;
    const int64_t slices = kk > 0 ? (kk + KT - 1) / KT : 0;
    LoadA la;
    LoadB lb;
    if (slices > 0) {
        const int k_left = kk < KT ? static_cast<int>(kk) : KT;
        la.load(a_base, p.a_rs, p.a_cs, w.rows_a, k_left);
        lb.load(b_base, p.b_cs, p.b_rs, w.rows_b, k_left);
        la.store(lds_a(0));
        lb.store(lds_b(0));
        __syncthreads();
    }
    for (int64_t s = 0; s < slices; ++s) {
        const int cur = static_cast<int>(s & 1);
        const bool more = s + 1 < slices;
        if (more) {
            const int64_t k_next = (s + 1) * KT;
            const int k_left = kk - k_next < KT ? static_cast<int>(kk - k_next) : KT;
            la.load(a_base + (s + 1) * a_step, p.a_rs, p.a_cs, w.rows_a, k_left);
            lb.load(b_base + (s + 1) * b_step, p.b_cs, p.b_rs, w.rows_b, k_left);
        }
        slice_mfma<LoadA, LoadB, KT, FM, FN, WM, WN, WAVES_K>(acc, lds_a(cur), lds_b(cur), wave_m,
                                                                wave_n, wave_k, half, r32);
        if (more) {
            la.store(lds_a(cur ^ 1));
            lb.store(lds_b(cur ^ 1));
        }
        __syncthreads();
    }

    if constexpr (WAVES_K > 1) {
        // The depth loop ended with a barrier, so the LDS tiles are free: sets 1.. park their
        // accumulators there (lane-contiguous), set 0 adds them in set order.
        constexpr int kPerWave = FM * FN * 16 * 64;
        static_assert((WAVES_K - 1) * WAVES_M * WAVES_N * kPerWave <=
                          2 * (LoadA::kFloats + LoadB::kFloats),
                      "the partial accumulators fit in the tiles' LDS");
        if (wave_k > 0) {
            float* mine = smem + ((wave_k - 1) * WAVES_M * WAVES_N + wave_mn) * kPerWave;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        mine[((i * FN + j) * 16 + e) * 64 + lane] = acc[i][j][e];
                    }
                }
            }
        }
        __syncthreads();
        if (wave_k > 0) {
            return;
        }
#pragma unroll
        for (int ws = 1; ws < WAVES_K; ++ws) {
            const float* theirs = smem + ((ws - 1) * WAVES_M * WAVES_N + wave_mn) * kPerWave;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        acc[i][j][e] += theirs[((i * FN + j) * 16 + e) * 64 + lane];
                    }
                }
            }
        }
    }
    finish_tile<BM, BN, WM, WN, FM, FN>(acc, p, w, wave_m, wave_n, half, r32,
                                        gelu_math::kExp2Table);
}

// ---- the direct-to-LDS form ---------------------------------------------------------------------

// Global -> LDS copy of one operand slice by buffer loads that write LDS (buffer_load ... lds):
// lane L of a wave-instruction lands its V floats at the instruction's LDS base + L * V floats, so
// each instruction fills 64 * V consecutive floats of the slice's LDS image (the layout of
// SliceLoader, so the fragments read it unchanged) and its lanes gather them from wherever they
// live. No register holds the slice, so 4-byte loads (operands that 16-byte loads cannot read)
// cost no registers and need no staging copy. The instructions are split over the waves in
// contiguous blocks.
//
// Addressing: a buffer resource per slice at the slice's first element, and a 32-bit byte offset
// per lane. A lane whose element is outside the matrix (or is a pad float of the layout) gets an
// offset at the resource's record limit, which the buffer unit answers with zeros without reading
// memory. Every in-range byte of a slice must lie below 2^30 bytes from its first element: the
// host checks the strides (direct_slices_fit) before it picks this loader.
constexpr uint32_t kDirectLimit = 0x80000000u;

// HOIST: keep the K-major offsets in registers across the depth loop (one per instruction of a
// wave); otherwise they are worked out at every issue (the choice for two 4-byte K-major
// operands, whose 18 offsets together spilled).
template <int ROWS, int KT, bool KMAJ, int V, int THREADS, bool HOIST = true>
struct DirectSliceLoader {
    static constexpr int kPitch = KMAJ ? KT + 4 : ROWS + 8;
    static constexpr int kFloats = KMAJ ? ROWS * (KT + 4) : KT * (ROWS + 8);
    // K-major: the whole image, pads included; otherwise ROWS / (64 V) instructions per depth.
    static constexpr int kPerLine = KMAJ ? 1 : ROWS / (64 * V);
    static constexpr int kInstr = KMAJ ? kFloats / (64 * V) : KT * kPerLine;
    static constexpr int kWaves = THREADS / 64;
    static constexpr int kPerWave = (kInstr + kWaves - 1) / kWaves;
    static_assert(!KMAJ || kFloats % (64 * V) == 0, "the image is a whole number of instructions");
    static_assert(KMAJ || ROWS % (64 * V) == 0, "a depth line is a whole number of instructions");
    static_assert(kPitch % V == 0, "a chunk of V floats never crosses a line of the image");

    // This lane's byte offsets, fixed for the whole depth loop. K-major: one per instruction of
    // this wave (element (row, depth) of the image position it fills; a pad takes depth KT - V of
    // its row, in range whenever the slice is). Otherwise: the lane's offset along a depth line
    // (the line and the instruction's place in it come as the scalar offset).
    uint32_t off[KMAJ && HOIST ? kPerWave : 1];
    uint32_t row_bytes, k_bytes;
    int rows; // rows of the tile inside the matrix (at most ROWS), fixed for the depth loop

    // The K-major offset of this lane in instruction j of this wave; the limit for a row outside
    // the matrix.
    __device__ __forceinline__ uint32_t kmaj_offset(int j) const {
        const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / 64));
        const int f = ((wave * kPerWave + j) * 64 + static_cast<int>(__lane_id())) * V;
        const int row = f / kPitch;
        const int at = f - row * kPitch;
        const int d = at < KT ? at : KT - V;
        return row < rows ? static_cast<uint32_t>(row) * row_bytes + static_cast<uint32_t>(d) * 4u
                          : kDirectLimit;
    }

    __device__ __forceinline__ DirectSliceLoader(int64_t row_stride, int64_t k_stride,
                                                 int rows_inside)
        : rows(rows_inside) {
        row_bytes = static_cast<uint32_t>(row_stride) * 4u;
        k_bytes = static_cast<uint32_t>(k_stride) * 4u;
        if constexpr (KMAJ && HOIST) {
#pragma unroll
            for (int j = 0; j < kPerWave; ++j) {
                off[j] = kmaj_offset(j);
            }
        } else if constexpr (!KMAJ) {
            off[0] = static_cast<uint32_t>(static_cast<int>(__lane_id()) * V) * 4u;
        } else {
            off[0] = 0u;
        }
    }

    // One wave-instruction: lane L's V floats from byte voffset + soffset of the resource land at
    // dst + L * V floats. (No immediate offset: the hardware adds it to the LDS address too.)
    __device__ __forceinline__ static void load(__amdgpu_buffer_rsrc_t rsrc, float* dst,
                                                uint32_t voffset, uint32_t soffset) {
        if constexpr (V == 4) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, static_cast<int>(voffset),
                                                     static_cast<int>(soffset), 0, 0);
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 4, static_cast<int>(voffset),
                                                     static_cast<int>(soffset), 0, 0);
        }
    }

    // base: element (row 0, depth 0) of the slice; k_left: depths inside (a multiple of V when
    // k is the unit-stride dimension). A full-depth slice uses the fixed offsets, whose rows
    // outside the matrix already point at the limit (K-major), or compares each lane's row (a
    // depth line; no division, and only in a tile with rows outside). A partial-depth slice (the
    // last) works out each lane's element and sends the ones outside to the limit.
    __device__ __forceinline__ void issue(float* lds, const float* base, int k_left) const {
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(base), 0, static_cast<int>(kDirectLimit - 1), kBufferWord3);
        const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / 64));
        const int lane = static_cast<int>(__lane_id());
        if (k_left >= KT) {
#pragma unroll
            for (int j = 0; j < kPerWave; ++j) {
                const int instr = wave * kPerWave + j;
                if (kInstr % kWaves != 0 && instr >= kInstr) {
                    break; // uniform: this wave's block ended
                }
                if constexpr (KMAJ) {
                    load(rsrc, lds + instr * 64 * V, HOIST ? off[HOIST ? j : 0] : kmaj_offset(j),
                         0u);
                } else {
                    // The line and the instruction's place in it come as the scalar offset (the
                    // immediate offset would move the LDS destination as well). A lane outside
                    // the matrix sends its offset to the limit; the scalar part stays below 2^30,
                    // so the sum does not wrap back into the record.
                    const int line = instr / kPerLine;
                    const int q = instr % kPerLine;
                    uint32_t voffset = off[0];
                    if (rows < ROWS) {
                        voffset = q * 64 * V + lane * V < rows ? voffset : kDirectLimit;
                    }
                    load(rsrc, lds + line * kPitch + q * 64 * V, voffset,
                         static_cast<uint32_t>(line) * k_bytes +
                             static_cast<uint32_t>(q * 64 * V * 4));
                }
            }
            return;
        }
        const int rows_left = rows;
        const int depth_end = k_left < KT ? k_left : KT; // depths of the slice inside the matrix
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int instr = wave * kPerWave + j;
            if (kInstr % kWaves != 0 && instr >= kInstr) {
                break;
            }
            uint32_t offset;
            float* dst;
            if constexpr (KMAJ) {
                // line = row, at = depth (at >= KT: a pad).
                const int f = (instr * 64 + lane) * V;
                const int row = f / kPitch;
                const int at = f - row * kPitch;
                const bool inside = row < rows_left && at < depth_end;
                offset = inside ? static_cast<uint32_t>(row) * row_bytes +
                                      static_cast<uint32_t>(at) * 4u
                                : kDirectLimit;
                dst = lds + instr * 64 * V;
            } else {
                // line = depth (uniform per instruction), at = row.
                const int line = instr / kPerLine;
                const int row = (instr % kPerLine) * 64 * V + lane * V;
                const bool inside = line < depth_end && row < rows_left;
                offset = inside ? static_cast<uint32_t>(line) * k_bytes +
                                      static_cast<uint32_t>(row) * 4u
                                : kDirectLimit;
                dst = lds + line * kPitch + (instr % kPerLine) * 64 * V;
            }
            load(rsrc, dst, offset, 0u);
        }
    }
};

// Direct-to-LDS copy of an M/N-major slice whose lines (KT of them, ROWS floats each, padded to
// ROWS + 8) are narrower than one wave-instruction (ROWS = 64): the image is filled as one run
// of floats, each lane's 4 floats (16 bytes, within one line) from wherever they live. The last
// instruction may run past the image, so the LDS buffer holds kAlloc floats. Elements outside the
// matrix and the pads get an offset past the record limit and load zeros.
template <int ROWS, int KT, int THREADS> struct DirectNarrowLoader {
    static constexpr int kPitch = ROWS + 8;
    static constexpr int kFloats = KT * kPitch;
    static constexpr int kInstr = (kFloats + 255) / 256;
    static constexpr int kAlloc = kInstr * 256;
    static constexpr int kWaves = THREADS / 64;
    static constexpr int kPerWave = (kInstr + kWaves - 1) / kWaves;
    uint32_t off[kPerWave]; // this lane's offsets in a full-depth slice (the limit outside)
    uint32_t k_bytes;

    // (line, position) of this lane's 4 floats in instruction j of this wave; false past the
    // image.
    __device__ __forceinline__ static bool place(int j, int& line, int& at) {
        const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / 64));
        const int f = ((wave * kPerWave + j) * 64 + static_cast<int>(__lane_id())) * 4;
        line = f / kPitch;
        at = f - line * kPitch;
        return f < kFloats;
    }

    // rows_inside: rows of the tile inside the matrix (at most ROWS); the others load zeros.
    __device__ __forceinline__ DirectNarrowLoader(int64_t k_stride, int rows_inside) {
        k_bytes = static_cast<uint32_t>(k_stride) * 4u;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            int line, at;
            const bool in_image = place(j, line, at);
            off[j] = in_image && at < ROWS && at < rows_inside
                         ? static_cast<uint32_t>(line) * k_bytes + static_cast<uint32_t>(at) * 4u
                         : kDirectLimit;
        }
    }

    // base: element (depth 0, row 0) of the slice; k_left as DirectSliceLoader's. Only a
    // partial-depth slice (the last) works out each lane's depth line.
    __device__ __forceinline__ void issue(float* lds, const float* base, int k_left) const {
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(base), 0, static_cast<int>(kDirectLimit - 1), kBufferWord3);
        const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / 64));
        const bool whole = k_left >= KT;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int instr = wave * kPerWave + j;
            if (kInstr % kWaves != 0 && instr >= kInstr) {
                break; // uniform: this wave's block ended
            }
            uint32_t offset = off[j];
            if (!whole) {
                int line, at;
                place(j, line, at);
                offset = line < k_left ? offset : kDirectLimit;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds + instr * 256, 16,
                                                     static_cast<int>(offset), 0, 0, 0);
        }
    }
};


// Whether a loader declares kAlloc (the narrow loader's buffer size).
template <typename L, typename = void> struct has_alloc : std::false_type {};
template <typename L> struct has_alloc<L, std::void_t<decltype(L::kAlloc)>> : std::true_type {};

// LDS floats a direct loader's buffer holds: the image, or for the narrow loader the whole
// instructions that fill it (the last may run past the image).
template <typename L> constexpr int direct_alloc() {
    if constexpr (has_alloc<L>::value) {
        return L::kAlloc;
    } else {
        return L::kFloats;
    }
}

// A direct loader from the operand's strides: along its rows (M for A, N for B) and along k. The
// narrow loader takes only the k stride (its lines are depth lines).
template <typename L, bool NARROW>
__device__ __forceinline__ L make_direct_loader(int64_t row_stride, int64_t k_stride, int rows) {
    if constexpr (NARROW) {
        return L(k_stride, rows);
    } else {
        return L(row_stride, k_stride, rows);
    }
}

// The 256x256 tile (16 wavefronts of 64x64) with direct-to-LDS slices. The depth loop is
// unrolled by two so each half knows at compile time which buffer it reads and which it fills;
// the copy of slice s + 1 is issued before slice s's MFMAs and waited for (vmcnt 0) before the
// barrier that ends the slice. Within a slice each wavefront reads group g + 1's fragments
// before group g's MFMAs (two register sets), and the slice's last group is held back across
// the barrier: its fragments are read before it (so the buffer may be refilled), its MFMAs run
// after it while the next slice's first fragments are read. Without the hold-back every
// wavefront waited after each barrier for its first reads, with the 16 wavefronts reading at
// once. Taken with both operands K-major (each fragment one 16-byte LDS read): configs[2] 972 ->
// 960 us. With an M/N-major operand it measured slower (4096^3 NN 950 -> 959 us, the MLP's
// rectangle 267 -> 269), so those take each slice's groups in order with no hold-back. Same
// arithmetic as sgemm_kernel, so the same bits.
template <int BM, int BN, int KT, int WAVES_M, int WAVES_N, bool AK, bool BK, int VA, int VB>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void sgemm_direct_kernel(GemmParams p) {
    constexpr int THREADS = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int FM = WM / 32;
    constexpr int FN = WN / 32;
    static_assert(KT % 8 == 0 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
    // Two 4-byte K-major operands: 18 hoisted offsets do not fit beside the accumulators.
    constexpr bool kHoist = !(AK && BK && VA == 1 && VB == 1);
    // An M/N-major operand whose lines are narrower than one 256-float wave-instruction (the
    // 64x64 and 128x128 tiles) is filled as one run of 16-byte pieces over its padded image
    // (DirectNarrowLoader, pitch ROWS + 8, the fragment reads' pitch).
    constexpr bool kNarrowA = !AK && BM < 256;
    constexpr bool kNarrowB = !BK && BN < 256;
    static_assert((!kNarrowA || VA == 4) && (!kNarrowB || VB == 4),
                  "narrow lines are copied in 16-byte pieces");
    using LoadA = std::conditional_t<kNarrowA, DirectNarrowLoader<BM, KT, THREADS>,
                                     DirectSliceLoader<BM, KT, AK, VA, THREADS, kHoist>>;
    using LoadB = std::conditional_t<kNarrowB, DirectNarrowLoader<BN, KT, THREADS>,
                                     DirectSliceLoader<BN, KT, BK, VB, THREADS, kHoist>>;
    using FragA = SliceLoader<BM, KT, AK, VA, THREADS>;
    using FragB = SliceLoader<BN, KT, BK, VB, THREADS>;
    static_assert(LoadA::kFloats == FragA::kFloats && LoadB::kFloats == FragB::kFloats &&
                      LoadA::kPitch == FragA::kPitch && LoadB::kPitch == FragB::kPitch,
                  "one LDS image");
    // The narrow loader's last instruction may run past the image.
    constexpr int kAllocA = direct_alloc<LoadA>();
    constexpr int kAllocB = direct_alloc<LoadB>();
    // One LDS object per buffer: the compiler tells LDS objects apart, so it sees that the copy
    // into one buffer does not write the one the MFMAs read (within one object it would wait for
    // the copy to land before the first LDS read of every slice).
    __shared__ __align__(16) float tile_a0[kAllocA];
    __shared__ __align__(16) float tile_a1[kAllocA];
    __shared__ __align__(16) float tile_b0[kAllocB];
    __shared__ __align__(16) float tile_b1[kAllocB];
    // The tanh gelu's exp table, copied into LDS: the epilogue's per-lane reads of it then wait
    // on the LDS counter alone. From global memory, each value's wait for its table load would
    // also wait for the output stores issued before it (one counter covers both).
    __shared__ double gelu_table[64];
    if (p.act == MFR_ACT_GELU_TANH && threadIdx.x < 64) {
        gelu_table[threadIdx.x] = gelu_math::kExp2Table[threadIdx.x];
    }

    const TileWork w = tile_work<BM, BN>(p);
    const float* a_base = p.a + w.off_a + w.m0 * p.a_rs + w.k_begin * p.a_cs;
    const float* b_base = p.b + w.off_b + w.n0 * p.b_cs + w.k_begin * p.b_rs;
    const int64_t a_step = KT * p.a_cs;
    const int64_t b_step = KT * p.b_rs;

    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    const int wave_m = wave / WAVES_N;
    const int wave_n = wave % WAVES_N;
    const int half = lane / 32;
    const int r32 = lane % 32;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                acc[i][j][e] = 0.0f;
            }
        }
    }

    // Fragments of one 8-deep group in two register sets: set (g & 1) for group g of a slice.
    constexpr int KG = KT / 8;
    static_assert(KG % 2 == 0, "a slice's first group takes register set 0");
    [[maybe_unused]] float fa[2][FM][4], fb[2][FN][4];
    // The slice lambdas capture the accumulators by reference and are always inlined: one left
    // as a call (deep slices make them long) would keep the accumulators in scratch memory.
    const auto frags = [&](int set, const float* sa, const float* sb, int g)
                           __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            FragA::fragment(sa, wave_m * WM + i * 32 + r32, g, half, fa[set][i]);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            FragB::fragment(sb, wave_n * WN + j * 32 + r32, g, half, fb[set][j]);
        }
    };
    const auto mfmas = [&](int set) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[set][i][st],
                                                                      fb[set][j][st], acc[i][j],
                                                                      0, 0, 0);
                }
            }
        }
    };
    // Groups 0 .. KG - 2 of the slice in (sa, sb), each after the next group's reads (the
    // scheduling barriers keep the reads ahead of the MFMAs that do not need them). Two groups
    // per step, so each names its register set as a constant even where the loop stays rolled
    // (a set index known only at run time puts both sets in scratch memory).
    const auto body = [&](const float* sa, const float* sb) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g + 1 < KG; g += 2) {
            frags(1, sa, sb, g + 1);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(0);
            __builtin_amdgcn_sched_barrier(0);
            if (g + 2 < KG) {
                frags(0, sa, sb, g + 2);
                __builtin_amdgcn_sched_barrier(0);
                mfmas(1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    // After the slice barrier: the next slice's first fragments, then the held-back last group.
    const auto cross = [&](const float* na, const float* nb) __attribute__((always_inline)) {
        frags(0, na, nb, 0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas((KG - 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
    };

    // Slices are taken in pairs, buffer 0 then buffer 1, with no exit between the two halves (an
    // exit there splits the accumulators' live ranges and they spill). An odd count gets one
    // more slice past the end, all of whose elements are outside the matrix: the buffer unit
    // loads zeros, and adding zero products leaves every sum as it was.
    const int64_t kk = w.kk;
    const int64_t slices = kk > 0 ? (kk + KT - 1) / KT : 0;
    const auto k_left_of = [&](int64_t s) {
        const int64_t left = kk - s * KT;
        return left <= 0 ? 0 : left < KT ? static_cast<int>(left) : KT;
    };
    const LoadA load_a = make_direct_loader<LoadA, kNarrowA>(p.a_rs, p.a_cs, w.rows_a);
    const LoadB load_b = make_direct_loader<LoadB, kNarrowB>(p.b_cs, p.b_rs, w.rows_b);
    constexpr bool kHold = AK && BK;
    if (slices > 0) {
        load_a.issue(tile_a0, a_base, k_left_of(0));
        load_b.issue(tile_b0, b_base, k_left_of(0));
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if constexpr (kHold) {
            frags(0, tile_a0, tile_b0, 0);
        }
    }
    for (int64_t s = 0; s < slices; s += 2) {
        // Slice s from buffer 0; slice s + 1 (zeros past the end) into buffer 1, whose last
        // reads came before the previous barrier.
        load_a.issue(tile_a1, a_base + (s + 1) * a_step, k_left_of(s + 1));
        load_b.issue(tile_b1, b_base + (s + 1) * b_step, k_left_of(s + 1));
        if constexpr (kHold) {
            body(tile_a0, tile_b0);
        } else {
            slice_mfma<FragA, FragB, KT, FM, FN, WM, WN, 1>(acc, tile_a0, tile_b0, wave_m, wave_n,
                                                             0, half, r32);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if constexpr (kHold) {
            cross(tile_a1, tile_b1);
        }
        // Slice s + 1 from buffer 1; slice s + 2 into buffer 0 (all of whose reads came before
        // the barrier above).
        if (s + 2 < slices) {
            load_a.issue(tile_a0, a_base + (s + 2) * a_step, k_left_of(s + 2));
            load_b.issue(tile_b0, b_base + (s + 2) * b_step, k_left_of(s + 2));
        }
        if constexpr (kHold) {
            body(tile_a1, tile_b1);
        } else {
            slice_mfma<FragA, FragB, KT, FM, FN, WM, WN, 1>(acc, tile_a1, tile_b1, wave_m, wave_n,
                                                             0, half, r32);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if constexpr (kHold) {
            cross(tile_a0, tile_b0); // past the last slice the fragments read here go unused
        }
    }
    if (slices == 0) {
        __syncthreads(); // the gelu table's copy (no slice barrier has made it visible)
    }
    finish_tile<BM, BN, WM, WN, FM, FN>(acc, p, w, wave_m, wave_n, half, r32, gelu_table);
}

// ---- the paired form: 64 columns of an N-major B ----------------------------------------------

// The 128x64 tile on a K-major A and an N-major B, both read by 16-byte direct-to-LDS loads:
// attention's P V (128 x [1024 x 1024] x [1024 x 64]). Four wavefronts of 32 rows x all 64
// columns. B's N-major fragments would take four 4-byte LDS reads per column block and depth
// group; here lane l's two accumulator blocks hold the column pair 2 (l % 32) and 2 (l % 32) + 1,
// so one 8-byte read feeds both blocks' MFMAs: 5 LDS reads per 8 MFMAs instead of 9. The depth
// order is the tile kernels' (the same sums, bit for bit). Double-buffered 32-deep slices, the
// copy of slice s + 1 issued before slice s's MFMAs and waited for before the barrier that ends
// it (no stores in the loop). The epilogue writes the paired layout (finish_tile, JS = 1). KT is
// the depth slice (32; split-K ranges are multiples of it).
// Config 5's P V on one MI355X: 165.7-169.6 us against 181.6-184.0 us for the register-copy
// 128x64 kernel (one process each).
template <int KT>
__global__ __launch_bounds__(256) void sgemm_pair_kernel(GemmParams p) {
    constexpr int BM = 128, BN = 64, THREADS = 256;
    using LoadA = DirectSliceLoader<BM, KT, true, 4, THREADS>;
    using LoadB = DirectNarrowLoader<BN, KT, THREADS>;
    using FragA = SliceLoader<BM, KT, true, 4, THREADS>;
    constexpr int PB = LoadB::kPitch;
    __shared__ __align__(16) float tile_a0[LoadA::kFloats];
    __shared__ __align__(16) float tile_a1[LoadA::kFloats];
    __shared__ __align__(16) float tile_b0[LoadB::kAlloc];
    __shared__ __align__(16) float tile_b1[LoadB::kAlloc];
    __shared__ double gelu_table[64];
    if (p.act == MFR_ACT_GELU_TANH && threadIdx.x < 64) {
        gelu_table[threadIdx.x] = gelu_math::kExp2Table[threadIdx.x];
    }

    const TileWork w = tile_work<BM, BN>(p);
    const float* a_base = p.a + w.off_a + w.m0 * p.a_rs + w.k_begin * p.a_cs;
    const float* b_base = p.b + w.off_b + w.n0 * p.b_cs + w.k_begin * p.b_rs;
    const int64_t a_step = KT * p.a_cs;
    const int64_t b_step = KT * p.b_rs;
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    const int half = lane / 32;
    const int r32 = lane % 32;

    floatx16 acc[1][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            acc[0][j][e] = 0.0f;
        }
    }
    const auto slice = [&](const float* sa, const float* sb) {
#pragma unroll
        for (int g = 0; g < KT / 8; ++g) {
            float fa[4];
            FragA::fragment(sa, wave * 32 + r32, g, half, fa);
            float2 fb[4];
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                fb[st] = *reinterpret_cast<const float2*>(sb + (8 * g + 4 * half + st) * PB +
                                                          2 * r32);
            }
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[st], fb[st].x, acc[0][0], 0,
                                                                 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[st], fb[st].y, acc[0][1], 0,
                                                                 0, 0);
            }
        }
    };

    // Slices in pairs (buffer 0 then 1) with no exit between the halves; an odd count runs one
    // slice past the end, which loads zeros and adds nothing (as sgemm_direct_kernel).
    const int64_t kk = w.kk;
    const int64_t slices = kk > 0 ? (kk + KT - 1) / KT : 0;
    const auto k_left_of = [&](int64_t s) {
        const int64_t left = kk - s * KT;
        return left <= 0 ? 0 : left < KT ? static_cast<int>(left) : KT;
    };
    const LoadA load_a(p.a_rs, p.a_cs, w.rows_a);
    const LoadB load_b(p.b_rs, w.rows_b);
    if (slices > 0) {
        load_a.issue(tile_a0, a_base, k_left_of(0));
        load_b.issue(tile_b0, b_base, k_left_of(0));
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    for (int64_t s = 0; s < slices; s += 2) {
        load_a.issue(tile_a1, a_base + (s + 1) * a_step, k_left_of(s + 1));
        load_b.issue(tile_b1, b_base + (s + 1) * b_step, k_left_of(s + 1));
        slice(tile_a0, tile_b0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (s + 2 < slices) {
            load_a.issue(tile_a0, a_base + (s + 2) * a_step, k_left_of(s + 2));
            load_b.issue(tile_b0, b_base + (s + 2) * b_step, k_left_of(s + 2));
        }
        slice(tile_a1, tile_b1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (slices == 0) {
        __syncthreads(); // the gelu table's copy
    }
    finish_tile<BM, BN, 32, BN, 1, 2, 1>(acc, p, w, wave, 0, half, r32, gelu_table);
}

} // namespace mfr::gemm
