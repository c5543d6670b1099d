// fp32 GEMM on the gfx950 fp32 matrix cores, with a fused epilogue (include/mfr_rocm.h,
// mfr_sgemm):
//
//   C[b] = act( fl( fl( fl(alpha * op(A[b]) op(B[b])) + fl(beta * C0[b]) ) + bias ) )
//
// Design (one workgroup = 256 threads = 4 wavefronts of 64):
//   - The workgroup computes a BM x BN tile of C; its wavefronts form a WAVES_M x WAVES_N grid,
//     each owning a (BM/WAVES_M) x (BN/WAVES_N) sub-tile held in 32x32 accumulator blocks of
//     v_mfma_f32_32x32x2_f32 (16 fp32 accumulators per lane per block).
//   - The depth is walked in slices of KT. Each slice of A (BM x KT) and B (KT x BN) is loaded
//     from global memory into registers one slice ahead, then written to the other half of a
//     double-buffered LDS tile, so one barrier per slice separates reads from writes.
//   - Operand layout in LDS follows the operand's layout in memory, so the copy never
//     transposes: a "K-major" operand (unit stride along the depth) is stored [rows][KT+4] and
//     its MFMA fragments are single 16-byte LDS reads; an "M/N-major" operand (unit stride
//     along its rows) is stored [KT][rows+8] and read as four 4-byte LDS reads. The pads keep
//     both reads free of bank conflicts.
//   - Depth permutation: within each group of 8 depth indices, lanes 0-31 of the wavefront feed
//     depths 0-3 and lanes 32-63 depths 4-7 over four MFMA steps (step s uses depths s and
//     4+s). A and B use the same permutation, so the sum is unchanged; it is what lets a
//     K-major fragment be one 16-byte read.
//   - Tiles are handed out XCD-aware: hardware sends workgroup i to XCD i % 8, so consecutive
//     logical tiles are remapped onto the same XCD (sharing its L2), and the logical order walks
//     GROUP_M tile-rows at a time so concurrently running tiles share A and B panels.
//   - Edges (M, N, K not multiples of the tile) are zero-filled on load and masked on store.
#include "common.hpp"

#include <type_traits>

namespace {

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
};

constexpr int kThreads = 256;

// Global -> register -> LDS copy of one operand slice: ROWS rows (M for A, N for B) by KT depth.
// KMAJ: unit stride along the depth (element (r, p) at base + r*row_stride + p).
// otherwise: unit stride along the rows (element (r, p) at base + p*k_stride + r).
// V: 4 = 16-byte loads along the unit-stride dimension (its extent and the other stride are
// multiples of 4, the base 16-byte aligned), 1 = 4-byte loads.
template <int ROWS, int KT, bool KMAJ, int V> struct SliceLoader {
    static constexpr int kUnits = ROWS * KT / V;        // loads per slice
    static constexpr int kPerThread = kUnits / kThreads;
    static_assert(kUnits % kThreads == 0, "slice must split evenly over the workgroup");
    // LDS row pitch: [ROWS][KT+4] (K-major) or [KT][ROWS+8].
    static constexpr int kPitch = KMAJ ? KT + 4 : ROWS + 8;
    static constexpr int kFloats = KMAJ ? ROWS * (KT + 4) : KT * (ROWS + 8);

    using Vec = typename std::conditional<V == 4, float4, float>::type;
    Vec reg[kPerThread];

    // (row, depth) of this thread's i-th load, in elements.
    __device__ static void coords(int i, int& r, int& p) {
        const int u = static_cast<int>(threadIdx.x) + i * kThreads;
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
    __device__ void load(const float* base, int64_t row_stride, int64_t k_stride, int rows_left,
                         int k_left) {
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

    __device__ void store(float* lds) const {
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
    __device__ static void fragment(const float* lds, int row, int g, int half, float out[4]) {
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

template <int BM, int BN, int KT, int WAVES_M, int WAVES_N, bool AK, bool BK, int VA, int VB>
__global__ __launch_bounds__(kThreads) void sgemm_kernel(GemmParams p) {
    static_assert(WAVES_M * WAVES_N * 64 == kThreads, "4 wavefronts per workgroup");
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int FM = WM / 32; // 32x32 accumulator blocks per wavefront, along M
    constexpr int FN = WN / 32;
    static_assert(KT % 8 == 0 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
    using LoadA = SliceLoader<BM, KT, AK, VA>;
    using LoadB = SliceLoader<BN, KT, BK, VB>;
    __shared__ float smem[2 * (LoadA::kFloats + LoadB::kFloats)];
    // Buffer `which` (0 or 1) of each operand's double-buffered slice.
    auto lds_a = [&](int which) { return smem + which * LoadA::kFloats; };
    auto lds_b = [&](int which) { return smem + 2 * LoadA::kFloats + which * LoadB::kFloats; };

    // ---- which tile: XCD-aware remap, then grouped row-major order within the batch ----
    const int64_t tiles_per_batch = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
    const int64_t total = tiles_per_batch * p.batch_count;
    const int64_t hw = blockIdx.x;
    const int64_t per_xcd = total / 8;
    const int64_t logical = hw < per_xcd * 8 ? (hw % 8) * per_xcd + hw / 8 : hw;
    int64_t batch_index = logical / tiles_per_batch;
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

    const float* a_base = p.a + off_a + m0 * p.a_rs;
    const float* b_base = p.b + off_b + n0 * p.b_cs;
    // Per slice the bases advance by KT depths.
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

    const int64_t slices = (p.k + KT - 1) / KT;
    LoadA la;
    LoadB lb;
    if (slices > 0) {
        const int k_left = p.k < KT ? static_cast<int>(p.k) : KT;
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
            const int k_left = p.k - k_next < KT ? static_cast<int>(p.k - k_next) : KT;
            la.load(a_base + (s + 1) * a_step, p.a_rs, p.a_cs, rows_a, k_left);
            lb.load(b_base + (s + 1) * b_step, p.b_cs, p.b_rs, rows_b, k_left);
        }
        const float* sa = lds_a(cur);
        const float* sb = lds_b(cur);
#pragma unroll
        for (int g = 0; g < KT / 8; ++g) {
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

    // ---- epilogue: accumulator e of block (i, j) is C(row, col) with
    //      row = 32i + 8(e/4) + 4*half + e%4, col = 32j + lane%32 (v_mfma_f32_32x32x2_f32 layout)
    float* c_base = p.c + off_c;
    const float* c0_base = p.c0 != nullptr ? p.c0 + off_c0 : nullptr;
    const bool use_c0 = c0_base != nullptr && p.beta != 0.0f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t col = n0 + wave_n * WN + j * 32 + r32;
            if (col >= p.n) {
                continue;
            }
            const float bias = p.bias != nullptr ? p.bias[col] : 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t row = m0 + wave_m * WM + i * 32 + 8 * (e / 4) + 4 * half + e % 4;
                if (row >= p.m) {
                    continue;
                }
                float v = acc[i][j][e];
                if (p.alpha != 1.0f) {
                    v = p.alpha * v;
                }
                if (use_c0) {
                    const float scaled = p.beta * c0_base[row * p.c0_rs + col];
                    v = v + scaled;
                }
                if (p.bias != nullptr) {
                    v = v + bias;
                }
                c_base[row * p.c_rs + col] = mfr::dev::activate(v, p.act);
            }
        }
    }
}

// Tile configuration of the one kernel family built so far.
constexpr int kBM = 128, kBN = 128, kKT = 32, kWavesM = 2, kWavesN = 2, kGroupM = 8;

template <bool AK, bool BK, int VA, int VB>
void launch_tile(const GemmParams& p, unsigned blocks, hipStream_t stream) {
    sgemm_kernel<kBM, kBN, kKT, kWavesM, kWavesN, AK, BK, VA, VB>
        <<<blocks, kThreads, 0, stream>>>(p);
}

template <bool AK, bool BK>
void launch_vec(const GemmParams& p, int va, int vb, unsigned blocks, hipStream_t stream) {
    if (va == 4 && vb == 4) {
        launch_tile<AK, BK, 4, 4>(p, blocks, stream);
    } else if (va == 4) {
        launch_tile<AK, BK, 4, 1>(p, blocks, stream);
    } else if (vb == 4) {
        launch_tile<AK, BK, 1, 4>(p, blocks, stream);
    } else {
        launch_tile<AK, BK, 1, 1>(p, blocks, stream);
    }
}

// 16-byte loads are possible for an operand when its unit-stride extent and its other stride
// (and every batch stride) are multiples of 4 floats and its base is 16-byte aligned.
int vector_width(const float* base, int64_t extent, int64_t other_stride, int64_t other_extent,
                 const int64_t* bs, int dims) {
    if (!mfr::aligned16(base) || extent % 4 != 0) {
        return 1;
    }
    if (other_extent > 1 && other_stride % 4 != 0) {
        return 1;
    }
    for (int d = 0; d < dims; ++d) {
        if (bs[d] % 4 != 0) {
            return 1;
        }
    }
    return 4;
}

void run_sgemm(mfr_stream& s, const mfr_gemm_desc& d) {
    using mfr::require;
    require(d.m >= 0 && d.n >= 0 && d.k >= 0, "sgemm: negative dimension");
    require(d.batch_dims >= 0 && d.batch_dims <= MFR_MAX_BATCH_DIMS,
            "sgemm: batch_dims out of range");
    require(d.act == MFR_ACT_NONE || d.act == MFR_ACT_GELU_TANH || d.act == MFR_ACT_GELU_ERF,
            "sgemm: unknown activation");
    int64_t batch_count = 1;
    for (int i = 0; i < d.batch_dims; ++i) {
        require(d.batch[i] >= 0, "sgemm: negative batch size");
        batch_count *= d.batch[i];
    }
    if (d.m == 0 || d.n == 0 || batch_count == 0) {
        return;
    }
    require(d.c != nullptr, "sgemm: null c");
    require(d.m == 1 || d.c_rs >= d.n, "sgemm: c row stride smaller than n");
    GemmParams p{};
    p.a = d.a;
    p.b = d.b;
    p.c = d.c;
    p.c0 = d.c0;
    p.bias = d.bias;
    p.m = d.m;
    p.n = d.n;
    p.k = d.k;
    p.a_rs = d.a_rs;
    p.a_cs = d.a_cs;
    p.b_rs = d.b_rs;
    p.b_cs = d.b_cs;
    p.c_rs = d.c_rs;
    p.c0_rs = d.c0 != nullptr ? d.c0_rs : 0;
    p.batch_dims = d.batch_dims;
    for (int i = 0; i < d.batch_dims; ++i) {
        p.batch[i] = d.batch[i];
        p.a_bs[i] = d.a_bs[i];
        p.b_bs[i] = d.b_bs[i];
        p.c_bs[i] = d.c_bs[i];
        p.c0_bs[i] = d.c0 != nullptr ? d.c0_bs[i] : 0;
    }
    p.act = d.act;
    p.alpha = d.alpha;
    p.beta = d.beta;
    p.batch_count = batch_count;

    // A dimension of extent 1 is never stepped along, so its stride is free: pick the one that
    // gives the operand a unit stride.
    bool ak = true, bk = true;
    int va = 1, vb = 1;
    if (d.k > 0) {
        require(d.a != nullptr && d.b != nullptr, "sgemm: null a or b");
        if (p.k == 1 && p.a_cs != 1) p.a_cs = 1;
        if (p.m == 1 && p.a_cs != 1) p.a_rs = 1;
        if (p.k == 1 && p.b_rs != 1 && p.b_cs != 1) p.b_rs = 1;
        if (p.n == 1 && p.b_rs != 1) p.b_cs = 1;
        if (p.a_cs == 1) {
            ak = true;
        } else if (p.a_rs == 1) {
            ak = false;
        } else {
            throw mfr::Error(MFR_E_UNSUPPORTED, "sgemm: A needs a unit stride along a dimension");
        }
        if (p.b_rs == 1) {
            bk = true;
        } else if (p.b_cs == 1) {
            bk = false;
        } else {
            throw mfr::Error(MFR_E_UNSUPPORTED, "sgemm: B needs a unit stride along a dimension");
        }
        va = ak ? vector_width(p.a, p.k, p.a_rs, p.m, p.a_bs, p.batch_dims)
                : vector_width(p.a, p.m, p.a_cs, p.k, p.a_bs, p.batch_dims);
        vb = bk ? vector_width(p.b, p.k, p.b_cs, p.n, p.b_bs, p.batch_dims)
                : vector_width(p.b, p.n, p.b_rs, p.k, p.b_bs, p.batch_dims);
    }
    if (p.beta != 0.0f && p.c0 != nullptr) {
        require(p.m == 1 || p.c0_rs >= p.n, "sgemm: c0 row stride smaller than n");
    }
    const int64_t tiles_m = (p.m + kBM - 1) / kBM;
    const int64_t tiles_n = (p.n + kBN - 1) / kBN;
    const int64_t blocks = tiles_m * tiles_n * batch_count;
    require(tiles_m < (int64_t{1} << 30) && tiles_n < (int64_t{1} << 30) &&
                blocks < (int64_t{1} << 31),
            "sgemm: problem too large for one launch");
    p.tiles_m = static_cast<int32_t>(tiles_m);
    p.tiles_n = static_cast<int32_t>(tiles_n);
    p.group_m = kGroupM;
    const unsigned grid = static_cast<unsigned>(blocks);
    if (ak && bk) {
        launch_vec<true, true>(p, va, vb, grid, s.stream);
    } else if (ak) {
        launch_vec<true, false>(p, va, vb, grid, s.stream);
    } else if (bk) {
        launch_vec<false, true>(p, va, vb, grid, s.stream);
    } else {
        launch_vec<false, false>(p, va, vb, grid, s.stream);
    }
    mfr::check_launch("sgemm_kernel");
}

} // namespace

extern "C" {

int mfr_sgemm(mfr_stream_t stream, const mfr_gemm_desc* desc) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(desc != nullptr, "sgemm: null descriptor");
        run_sgemm(s, *desc);
    });
}

int mfr_sgemm_rm(mfr_stream_t stream, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
                 float alpha, const float* a, int64_t lda, const float* b, int64_t ldb, float beta,
                 const float* c0, float* c, int64_t ldc) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr_gemm_desc d{};
        d.m = m;
        d.n = n;
        d.k = k;
        d.a = a;
        // op(A) = A [m,k] stored row-major with lda, or A^T where A is stored [k,m].
        d.a_rs = trans_a ? 1 : lda;
        d.a_cs = trans_a ? lda : 1;
        d.b = b;
        d.b_rs = trans_b ? 1 : ldb;
        d.b_cs = trans_b ? ldb : 1;
        d.c = c;
        d.c_rs = ldc;
        d.c0 = c0;
        d.c0_rs = ldc;
        d.alpha = alpha;
        d.beta = beta;
        d.act = MFR_ACT_NONE;
        run_sgemm(s, d);
    });
}

} // extern "C"
