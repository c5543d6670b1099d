// Device code of the fp32 MFMA GEMM: the tile kernel and its operand loader. Included by
// gemm.hip (the C ABI entry points and tile selection). See gemm.hip for the design.
#pragma once

#include "common.hpp"

#include <type_traits>

namespace mfr::gemm {

typedef float floatx16 __attribute__((ext_vector_type(16)));

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
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                out[s] = lds[(8 * g + 4 * half + s) * kPitch + row];
            }
        }
    }
};

// Writes a wavefront's accumulators: block (i, j), element e is C(row0 + 32i + 8(e/4) + e%4,
// col0 + 32j), as
//   C = act(fl(fl(fl(alpha * acc) + fl(beta * C0)) + bias))      (RAW: C = acc),
// the C0 term only when c0 is non-null and the bias only when p.bias is non-null, so the roundings
// are the reference's. alpha * acc is exact for alpha == 1. INTERIOR: every row and column is
// inside C (no checks). C0 == kC0Batched: c0 is non-null and a row-block's C0 values are all
// loaded before any is used, so the loads overlap; kC0None: no C0; kC0Checked: c0 checked per
// element (one copy of the code for both cases). STREAM: non-temporal stores.
enum { kC0None = 0, kC0Batched = 1, kC0Checked = 2 };
template <int FM, int FN, int ACT, bool INTERIOR, bool RAW, int C0, bool STREAM = false>
__device__ __forceinline__ void write_tile(const floatx16 (&acc)[FM][FN], float* c, int64_t c_rs,
                                           const float* c0, int64_t c0_rs, const GemmParams& p,
                                           int64_t row0, int64_t col0) {
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
                    const bool inside = INTERIOR || (col0 + 32 * j < p.n && row_i + dr < p.m);
                    c0v[j][e] = inside ? c0_i[dr * c0_rs + 32 * j] : 0.0f;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t col = col0 + 32 * j;
            if (!INTERIOR && col >= p.n) {
                continue;
            }
            const float bias = !RAW && p.bias != nullptr ? p.bias[col] : 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int dr = 8 * (e / 4) + e % 4;
                if (!INTERIOR && row_i + dr >= p.m) {
                    continue;
                }
                float v = acc[i][j][e];
                if constexpr (!RAW) {
                    v = p.alpha * v;
                    if constexpr (C0 == kC0Batched) {
                        const float scaled = p.beta * c0v[j][e];
                        v = v + scaled;
                    } else if constexpr (C0 == kC0Checked) {
                        if (c0 != nullptr) {
                            const float scaled = p.beta * c0[(row_i + dr) * c0_rs + col];
                            v = v + scaled;
                        }
                    }
                    if (p.bias != nullptr) {
                        v = v + bias;
                    }
                    if constexpr (ACT != MFR_ACT_NONE) {
                        v = mfr::dev::gelu(v, ACT);
                    }
                }
                if constexpr (STREAM) {
                    __builtin_nontemporal_store(v, &c_i[dr * c_rs + 32 * j]);
                } else {
                    c_i[dr * c_rs + 32 * j] = v;
                }
            }
        }
    }
}

// The epilogue for activation ACT. Without one it is dispatched on C0 and on whether the tile is
// interior; a gelu epilogue is one copy (its transcendental work outweighs the checks).
template <int FM, int FN, int ACT>
__device__ __forceinline__ void epilogue(const floatx16 (&acc)[FM][FN], float* c, int64_t c_rs,
                                         const float* c0, int64_t c0_rs, const GemmParams& p,
                                         int64_t row0, int64_t col0, bool interior) {
    if constexpr (ACT != MFR_ACT_NONE) {
        write_tile<FM, FN, ACT, false, false, kC0Checked>(acc, c, c_rs, c0, c0_rs, p, row0, col0);
    } else if (c0 != nullptr) {
        if (interior) {
            write_tile<FM, FN, ACT, true, false, kC0Batched>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                             col0);
        } else {
            write_tile<FM, FN, ACT, false, false, kC0Batched>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                              col0);
        }
    } else {
        if (interior && p.stream_c) {
            write_tile<FM, FN, ACT, true, false, kC0None, true>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                                col0);
        } else if (interior) {
            write_tile<FM, FN, ACT, true, false, kC0None>(acc, c, c_rs, c0, c0_rs, p, row0, col0);
        } else {
            write_tile<FM, FN, ACT, false, false, kC0None>(acc, c, c_rs, c0, c0_rs, p, row0,
                                                           col0);
        }
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

    // ---- which tile: XCD-aware remap, then grouped row-major order within the batch; the
    //      depth split is the outermost index ----
    const int64_t tiles_per_batch = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
    const int64_t tiles_per_split = tiles_per_batch * p.batch_count;
    const int64_t total = tiles_per_split * p.splits;
    const int64_t hw = blockIdx.x;
    const int64_t per_xcd = total / 8;
    const int64_t logical_all = hw < per_xcd * 8 ? (hw % 8) * per_xcd + hw / 8 : hw;
    const int64_t split = logical_all / tiles_per_split;
    const int64_t logical = logical_all - split * tiles_per_split;
    const int64_t batch_linear = logical / tiles_per_batch;
    int64_t batch_index = batch_linear;
    const int64_t t = logical % tiles_per_batch;
    const int64_t group_tiles = static_cast<int64_t>(p.group_m) * p.tiles_n;
    const int64_t group = t / group_tiles;
    const int64_t first_m = group * p.group_m;
    const int64_t rows_in_group =
        p.tiles_m - first_m < p.group_m ? p.tiles_m - first_m : p.group_m;
    const int64_t in_group = t % group_tiles;
    const int64_t tile_m = first_m + in_group % rows_in_group;
    const int64_t tile_n = in_group / rows_in_group;

    int64_t off_a = 0, off_b = 0, off_c = 0, off_c0 = 0;
    for (int d = p.batch_dims - 1; d >= 0; --d) {
        const int64_t idx = batch_index % p.batch[d];
        batch_index /= p.batch[d];
        off_a += idx * p.a_bs[d];
        off_b += idx * p.b_bs[d];
        off_c += idx * p.c_bs[d];
        off_c0 += idx * p.c0_bs[d];
    }
    const int64_t m0 = tile_m * BM;
    const int64_t n0 = tile_n * BN;
    const int rows_a = p.m - m0 < BM ? static_cast<int>(p.m - m0) : BM;
    const int rows_b = p.n - n0 < BN ? static_cast<int>(p.n - n0) : BN;

    // This workgroup's depth range [k_begin, k_begin + kk).
    const int64_t k_begin = split * p.k_per_split;
    const int64_t kk = p.k - k_begin < p.k_per_split ? p.k - k_begin : p.k_per_split;
    const float* a_base = p.a + off_a + m0 * p.a_rs + k_begin * p.a_cs;
    const float* b_base = p.b + off_b + n0 * p.b_cs + k_begin * p.b_rs;
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

    const int64_t slices = kk > 0 ? (kk + KT - 1) / KT : 0;
    LoadA la;
    LoadB lb;
    if (slices > 0) {
        const int k_left = kk < KT ? static_cast<int>(kk) : KT;
        la.load(a_base, p.a_rs, p.a_cs, rows_a, k_left);
        lb.load(b_base, p.b_cs, p.b_rs, rows_b, k_left);
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
            la.load(a_base + (s + 1) * a_step, p.a_rs, p.a_cs, rows_a, k_left);
            lb.load(b_base + (s + 1) * b_step, p.b_cs, p.b_rs, rows_b, k_left);
        }
        const float* sa = lds_a(cur);
        const float* sb = lds_b(cur);
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
        for (int w = 1; w < WAVES_K; ++w) {
            const float* theirs = smem + ((w - 1) * WAVES_M * WAVES_N + wave_mn) * kPerWave;
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

    // ---- epilogue: accumulator e of block (i, j) is C(row, col) with
    //      row = 32i + 8(e/4) + 4*half + e%4, col = 32j + lane%32 (v_mfma_f32_32x32x2_f32 layout)
    const int64_t row0 = m0 + wave_m * WM + 4 * half;
    const int64_t col0 = n0 + wave_n * WN + r32;
    const bool interior = m0 + BM <= p.m && n0 + BN <= p.n;
    if (p.partial != nullptr) {
        // Split-K: raw sums only, to partial[split][batch] (dense m x n).
        float* part = p.partial + (split * p.batch_count + batch_linear) * p.m * p.n;
        if (interior) {
            write_tile<FM, FN, MFR_ACT_NONE, true, true, kC0None>(acc, part, p.n, nullptr, 0, p,
                                                                  row0, col0);
        } else {
            write_tile<FM, FN, MFR_ACT_NONE, false, true, kC0None>(acc, part, p.n, nullptr, 0, p,
                                                                   row0, col0);
        }
        return;
    }
    float* c_base = p.c + off_c;
    const float* c0_base = p.c0 != nullptr && p.beta != 0.0f ? p.c0 + off_c0 : nullptr;
    // One activation per branch (uniform), so each epilogue is straight-line code: unrolled
    // over every accumulator, the three would not fit the instruction cache together.
    if (p.act == MFR_ACT_NONE) {
        epilogue<FM, FN, MFR_ACT_NONE>(acc, c_base, p.c_rs, c0_base, p.c0_rs, p, row0, col0,
                                       interior);
    } else if (p.act == MFR_ACT_GELU_TANH) {
        epilogue<FM, FN, MFR_ACT_GELU_TANH>(acc, c_base, p.c_rs, c0_base, p.c0_rs, p, row0, col0,
                                            interior);
    } else {
        epilogue<FM, FN, MFR_ACT_GELU_ERF>(acc, c_base, p.c_rs, c0_base, p.c0_rs, p, row0, col0,
                                           interior);
    }
}

} // namespace mfr::gemm
