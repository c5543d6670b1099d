// fp32 GEMM on the gfx950 fp32 matrix cores, with a fused epilogue (include/mfr_rocm.h,
// mfr_sgemm):
//
//   C[b] = act( fl( fl( fl(alpha * op(A[b]) op(B[b])) + fl(beta * C0[b]) ) + bias ) )
//
// Design (a workgroup of 4 or 16 wavefronts of 64 lanes; five MFMA tile shapes and a thin path,
// chosen per call with the split-K count and edge peeling, below):
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
//   - Operand staging: the 16-byte loads need an operand's lines (runs along its unit stride) to
//     start 16-byte aligned and hold a multiple of 4 floats. An operand that is not laid out so
//     (X[4093,1023] row-major) is copied first into the stream's workspace with its lines padded
//     to a multiple of 4 by zeros (stage_kernel); vector loads that reach past the end of a line
//     then read zeros of its own line, and the zeros add nothing to any sum. When a peeled strip
//     of at most 8 columns covers every row of such an A, the strip's launch writes the copy as
//     it reads A (strip_stage_kernel in thin_kernel.hpp), one launch instead of two.
//   - Direct-to-LDS slices (sgemm_direct_kernel, the 256x256 tile with a 4-byte operand): each
//     lane's buffer load writes its element into the LDS image itself, so 4-byte operands take
//     no registers and need no staging copy; elements outside the matrix get an offset past the
//     buffer's record limit and load as zeros. Its 16-byte form also replaces the register copy
//     on aligned operands. Under it AUTO stages only K-major 4-byte operands (whose in-place
//     runs of 32 floats touch twice the cache lines) and reads M/N-major ones in place.
//   - The epilogue applies the activation chosen once per workgroup, with copies for interior
//     tiles and for C0, so each copy is straight-line code (gemm_kernel.hpp, write_tile); the
//     tanh gelu's copies read its exp table from LDS and have no branch between elements.
//   - Split-K cuts a long depth into ranges run as workgroups of their own, reduced in order by
//     split_reduce_kernel; edge peeling runs a thin remainder of the output as launches of its
//     own; the thin path (thin_kernel.hpp) takes products with at most 8 output columns or rows.
#include "gemm_kernel.hpp"
#include "panel_kernel.hpp"
#include "thin_kernel.hpp"

#include <cstring>

#include <algorithm>
#include <cmath>

namespace {

using namespace mfr::gemm;

// ---- tile configurations ----------------------------------------------------------------------
//
// Five workgroup tiles (include/mfr_rocm.h, MFR_TILE_*). `tflops` is each tile's measured rate on
// the 4096^3 NT problem (one MI355X) and `occupancy` its resident workgroups per CU (LDS and
// registers); the automatic choice uses both.
struct TileInfo {
    int bm, bn, occupancy, waves;
    double tflops;
};
constexpr TileInfo kTiles[MFR_TILE_COUNT] = {
    {0, 0, 0, 0, 0.0},         // AUTO
    {256, 256, 1, 16, 135.3},  // 16 wavefronts of 64x64, depth slice 32
    {128, 128, 2, 4, 127.3},   // 4 wavefronts of 64x64, depth slice 32
    {128, 64, 5, 4, 114.9},    // 4 wavefronts of 64x32, depth slice 16
    {64, 128, 5, 4, 116.0},    // 4 wavefronts of 32x64, depth slice 16
    {64, 64, 4, 4, 111.4},     // 4 wavefronts of 32x32, depth slice 32
    {0, 0, 0, 0, 0.0},         // THIN (no tile; priced by thin_us)
    {0, 0, 0, 0, 0.0},         // PANEL (chosen by its own rule, panel_fits)
};
constexpr int kGroupM = 8;

int64_t tile_count(int tile, int64_t m, int64_t n, int64_t batch) {
    return ((m + kTiles[tile].bm - 1) / kTiles[tile].bm) *
           ((n + kTiles[tile].bn - 1) / kTiles[tile].bn) * batch;
}

// ---- split-K ------------------------------------------------------------------------------------
//
// A product with few output tiles and a long depth (256 x 256 x 16384) leaves most CUs idle. It
// is cut along the depth into `splits` ranges, each range a workgroup of its own writing raw sums
// to the workspace; split_reduce_kernel adds them in order and applies the epilogue.

constexpr int kMaxSplits = MFR_MAX_SPLITS;
constexpr int64_t kMinAutoDepth = 256;           // AUTO never cuts a range shorter than this
constexpr double kMaxPartialBytes = 1073741824.0; // AUTO keeps the partial sums under 1 GiB
constexpr double kReduceBytesPerUs = 4.0e6;       // split_reduce_kernel's HBM rate (bytes/us)
constexpr double kReduceLaunchUs = 4.0;           // its launch and ramp
// A tile's fixed cost (first slice's load latency, writing the tile out), in depth-equivalents
// of its MFMA work, shared among the workgroups a CU runs at once. Fit, with simd_efficiency, to
// the measured times of every tile and split count on 14 shapes (64^2 x 65536 .. 8192^2 x 1024).
constexpr double kTileOverheadDepth = 96.0;

// Depth of each range when `splits` are asked for: a multiple of 32, which every tile's depth
// slice divides, so no range starts inside a slice.
int64_t depth_per_split(int64_t k, int splits) {
    const int64_t per = (k + splits - 1) / splits;
    return (per + 31) / 32 * 32;
}

int splits_for(int64_t k, int64_t per) { return static_cast<int>((k + per - 1) / per); }

// Relative rate of a CU by how many wavefronts each SIMD holds: one alone hides no latency.
double simd_efficiency(int64_t waves_per_simd) {
    return waves_per_simd >= 3 ? 1.0 : waves_per_simd == 2 ? 0.9 : 0.85;
}

// Modelled time (us) of tile t with `splits` depth ranges of `per` each: the busiest CU's share
// of the tiles, each its depth plus the fixed overhead, at the tile's rate on 4096^3 (with the
// overhead taken out), scaled by its wavefronts per SIMD relative to that measurement; plus the
// reduce pass when split.
double modelled_us(int t, int64_t m, int64_t n, int64_t k, int64_t batch, int cus, int splits,
                   int64_t per, bool c0) {
    const TileInfo& info = kTiles[t];
    const int64_t count = tile_count(t, m, n, batch) * splits;
    const int64_t per_cu = (count + cus - 1) / cus;
    const int64_t concurrent = per_cu < info.occupancy ? per_cu : info.occupancy;
    // The 128x128 tile runs 8 wavefronts when no CU gets two (launch_layout). (The 64x64 tile
    // then runs 16, four sets sharing each depth slice, but is priced as its 4-wavefront form:
    // priced at 4 per SIMD, AUTO took it over split-K and the thin path where it is slower, e.g.
    // 512^3 16.2 against 14.1 us, the MLP's 4093 x 3 strip 19.1 against 7.9 us.)
    const int64_t waves = t == MFR_TILE_128x128 && count <= cus ? 8 : info.waves;
    const int64_t reference_waves = (4096 / info.bm) * (4096 / info.bn) / 256;
    const int64_t ref_concurrent =
        reference_waves < info.occupancy ? reference_waves : info.occupancy;
    const double efficiency = simd_efficiency(concurrent * waves / 4) /
                              simd_efficiency(ref_concurrent * info.waves / 4);
    const double depth = static_cast<double>(splits > 1 ? per : k);
    const double overhead = kTileOverheadDepth / static_cast<double>(concurrent);
    const double cu_flops_per_us = info.tflops * 1e6 / 256.0 *
                                   (4096.0 + kTileOverheadDepth / ref_concurrent) / 4096.0;
    double us = static_cast<double>(per_cu) * 2.0 * info.bm * info.bn * (depth + overhead) /
                (cu_flops_per_us * efficiency);
    if (splits > 1) {
        const double outputs = static_cast<double>(m) * n * batch;
        us += outputs * 4.0 * (2.0 * splits + (c0 ? 2.0 : 1.0)) / kReduceBytesPerUs +
              kReduceLaunchUs;
    }
    return us;
}

// ---- the thin path ---------------------------------------------------------------------------

constexpr double kThinBytesPerUs = 6.5e6; // its streaming rate (bytes/us) for one column
constexpr double kThinLaunchUs = 3.0;

// Whether the thin path takes an m x n product: n <= 8 with A read along k (ak), or m <= 8 with
// B read along k (bk). along_n: the first (C = A B row by row), else the transposed form.
bool thin_possible(int64_t m, int64_t n, bool ak, bool bk, bool* along_n = nullptr) {
    const bool by_rows = n <= kThinCols && ak;
    if (along_n != nullptr) {
        *along_n = by_rows;
    }
    return by_rows || (m <= kThinCols && bk);
}

// How the thin path will read B' (A in the transposed form), for thin_us: 2 = in pieces of
// C columns whatever the column count (a staged copy, lines zero-padded to a multiple of 4), 1 =
// in pieces when the column count is exactly 2, 4 or 8 (unit column stride, rows and batches
// 16-byte aligned), 0 = one load per value. launch_thin decides from the operand itself.
struct Plan;
int thin_b_layout(const GemmParams& p, const Plan& plan, int64_t m, int64_t n);

// Modelled time (us): every byte read or written once, at kThinBytesPerUs for one column; the
// kernel computes the columns rounded up to C = 1, 2, 4 or 8. Read one value at a time, B' costs
// a cache-line access per value, so C > 1 takes 0.75 * C times as long (16384^2 x 1: 168 us;
// 16384 x 4 x 4096: 125 us; 4096 x 8 x 1024: 22 us). Read in pieces, C = 2, 4 take 1.0 and 1.2
// times as long (16384 x 2 x 4096: 43 us; 16384 x 4 x 4096: 51 us; 65536 x 4 x 512: 25 us);
// C = 8 with B' staged in LDS 1.35 (16384 x 8 x 4096: 55.6 us; 65536 x 8 x 512: 31.6 us;
// 16384 x 8 x 1000: 15.3 us), 2.5 without (fewer than 16 rows). Slower in proportion with fewer
// than 1024 wavefronts.
double thin_us(int64_t m, int64_t n, int64_t k, int64_t batch, bool c0, bool ak, bool bk,
               int thin_b) {
    bool along_n = true;
    thin_possible(m, n, ak, bk, &along_n);
    const double rows = static_cast<double>(along_n ? m : n);
    const double cols = static_cast<double>(along_n ? n : m);
    const double rounded = cols <= 1 ? 1.0 : cols <= 2 ? 2.0 : cols <= 4 ? 4.0 : 8.0;
    const double bytes = 4.0 * batch * (rows * k + k * cols + rows * cols * (c0 ? 2.0 : 1.0));
    const bool pieces = rounded > 1.0 && (thin_b == 2 || (thin_b == 1 && cols == rounded));
    // 8 columns in pieces from kThinLdsMinRows rows: thin_dot_lds_kernel (B' staged in LDS).
    const bool lds = pieces && rounded == 8.0 && rows >= kThinLdsMinRows;
    const double waves =
        lds ? batch * std::ceil(rows / thin_lds_rows<kThinLdsWaves>()) * kThinLdsWaves
            : batch * std::ceil(rows / kThinDotRows) * kThinWaves;
    const double factor = rounded == 1.0 ? 1.0
                          : !pieces      ? 0.75 * rounded
                          : rounded == 2.0 ? 1.0
                          : rounded == 4.0 ? 1.2
                          : lds          ? 1.35
                                         : 2.5;
    return bytes / kThinBytesPerUs * factor * std::max(1.0, 1024.0 / waves) + kThinLaunchUs;
}

struct Choice {
    int tile = MFR_TILE_128x128;
    int splits = 1;      // depth ranges
    int64_t per = 0;     // depth of each (the last may be shorter); k when not split
    double us = 0.0;     // modelled time
};

// The automatic tile and split count (either may be fixed by the caller: tile != AUTO, splits !=
// 0). A short depth (K <= 128) is latency-bound per tile, so it takes the high-occupancy 128x64 /
// 64x128 tiles (the one padding the output less). Otherwise the pair with the least modelled
// time. The thin path competes where it
// can take the product (ak, bk: whether A and B are read along k) and no split is fixed.
// big_ok: whether the 256x256 tile can read the operands (big_tile_ok).
Choice choose(int64_t m, int64_t n, int64_t k, int64_t batch, int cus,
              int fixed_tile, int fixed_splits, bool c0, bool ak, bool bk, int thin_b,
              bool big_ok) {
    Choice best;
    best.per = k;
    if (fixed_tile == MFR_TILE_256x256 && !big_ok) {
        throw mfr::Error(MFR_E_UNSUPPORTED,
                         "sgemm: the 256x256 tile reads its slices with 32-bit offsets, and an "
                         "operand's strides put a slice more than 2^30 bytes across");
    }
    const bool thin = thin_possible(m, n, ak, bk) && fixed_splits <= 1;
    if (fixed_tile == MFR_TILE_THIN) {
        if (!thin) {
            throw mfr::Error(MFR_E_UNSUPPORTED,
                             "sgemm: the thin path takes n <= 8 with A read along k, or m <= 8 "
                             "with B read along k, and no split");
        }
        best.tile = MFR_TILE_THIN;
        best.us = thin_us(m, n, k, batch, c0, ak, bk, thin_b);
        return best;
    }
    if (fixed_splits > 0 && k > 0) {
        best.per = depth_per_split(k, fixed_splits);
        best.splits = splits_for(k, best.per);
        if (best.splits == 1) {
            best.per = k;
        }
    }
    if (fixed_tile == MFR_TILE_AUTO && best.splits == 1 && k <= 128) {
        const int64_t a = tile_count(MFR_TILE_128x64, m, n, batch) * 128 * 64;
        const int64_t b = tile_count(MFR_TILE_64x128, m, n, batch) * 64 * 128;
        best.tile = b < a ? MFR_TILE_64x128 : MFR_TILE_128x64;
        best.us = modelled_us(best.tile, m, n, k, batch, cus, 1, k, c0);
    } else {
        double best_us = 1e300;
        for (int t = 1; t < MFR_TILE_THIN; ++t) {
            if ((fixed_tile != MFR_TILE_AUTO && t != fixed_tile) ||
                (t == MFR_TILE_256x256 && !big_ok)) {
                continue;
            }
            if (fixed_splits > 0) {
                // Only the tile is open.
                const double us = modelled_us(t, m, n, k, batch, cus, best.splits, best.per, c0);
                if (us < best_us) {
                    best_us = us;
                    best.tile = t;
                    best.us = us;
                }
                continue;
            }
            int prev = 0;
            for (int want = 1; want <= kMaxSplits; ++want) {
                const int64_t per = want == 1 || k == 0 ? k : depth_per_split(k, want);
                const int splits = want == 1 || k == 0 ? 1 : splits_for(k, per);
                if (splits == prev) {
                    continue;
                }
                prev = splits;
                if (splits > 1 &&
                    (per < kMinAutoDepth ||
                     4.0 * splits * static_cast<double>(m) * n * batch > kMaxPartialBytes)) {
                    break;
                }
                const double us = modelled_us(t, m, n, k, batch, cus, splits, per, c0);
                if (us < best_us) {
                    best_us = us;
                    best.tile = t;
                    best.splits = splits;
                    best.per = per;
                    best.us = us;
                }
            }
        }
    }
    if (fixed_tile == MFR_TILE_AUTO && thin) {
        const double us = thin_us(m, n, k, batch, c0, ak, bk, thin_b);
        if (us < best.us) {
            best.tile = MFR_TILE_THIN;
            best.splits = 1;
            best.per = k;
            best.us = us;
        }
    }
    return best;
}

// C[b](i, j) = act(fl(fl(fl(alpha * sum_s partial[s][b](i, j)) + fl(beta * C0[b](i, j))) +
// bias[j])) for every output of a split-K product: the splits are added in order in fp32, then
// the epilogue of sgemm_kernel, with its roundings. Lines (batch, row) go over blockIdx.y,
// columns over blockIdx.x and the threads.
__global__ __launch_bounds__(256) void split_reduce_kernel(GemmParams p) {
    const int64_t lines = p.m * p.batch_count;
    const int64_t split_stride = lines * p.n;
    for (int64_t line = blockIdx.y; line < lines; line += gridDim.y) {
        const int64_t b = line / p.m;
        const int64_t row = line - b * p.m;
        int64_t rest = b, off_c = 0, off_c0 = 0;
        for (int d = p.batch_dims - 1; d >= 0; --d) {
            const int64_t index = rest % p.batch[d];
            rest /= p.batch[d];
            off_c += index * p.c_bs[d];
            off_c0 += index * p.c0_bs[d];
        }
        const float* part = p.partial + line * p.n;
        float* c_row = p.c + off_c + row * p.c_rs;
        const float* c0_row =
            p.c0 != nullptr && p.beta != 0.0f ? p.c0 + off_c0 + row * p.c0_rs : nullptr;
        for (int64_t col = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
             col < p.n; col += static_cast<int64_t>(gridDim.x) * blockDim.x) {
            float v = part[col];
            for (int32_t s = 1; s < p.splits; ++s) {
                v += part[s * split_stride + col];
            }
            if (p.alpha != 1.0f) {
                v = p.alpha * v;
            }
            if (c0_row != nullptr) {
                const float scaled = p.beta * c0_row[col];
                v = v + scaled;
            }
            if (p.bias != nullptr) {
                v = v + p.bias[col];
            }
            c_row[col] = mfr::dev::activate(v, p.act);
        }
    }
}

template <int BM, int BN, int KT, int WAVES_M, int WAVES_N, bool AK, bool BK, int WAVES_K = 1>
void launch_vec(const GemmParams& p, int va, int vb, unsigned blocks, hipStream_t stream) {
    constexpr int threads = WAVES_M * WAVES_N * WAVES_K * 64;
    if (va == 4 && vb == 4) {
        sgemm_kernel<BM, BN, KT, WAVES_M, WAVES_N, AK, BK, 4, 4, WAVES_K>
            <<<blocks, threads, 0, stream>>>(p);
    } else if (va == 4) {
        sgemm_kernel<BM, BN, KT, WAVES_M, WAVES_N, AK, BK, 4, 1, WAVES_K>
            <<<blocks, threads, 0, stream>>>(p);
    } else if (vb == 4) {
        sgemm_kernel<BM, BN, KT, WAVES_M, WAVES_N, AK, BK, 1, 4, WAVES_K>
            <<<blocks, threads, 0, stream>>>(p);
    } else {
        sgemm_kernel<BM, BN, KT, WAVES_M, WAVES_N, AK, BK, 1, 1, WAVES_K>
            <<<blocks, threads, 0, stream>>>(p);
    }
}

// one_per_cu: no CU gets more than one workgroup. The 128x128 tile then runs 8 wavefronts of
// 64x32 (2 per SIMD) instead of 4 of 64x64: 2048^3 145 against 155 us. With two workgroups per
// CU the 4 wavefronts are faster (4096^3 1075 against 1105 us). Unsplit, the 128x128 tile
// then runs 16 wavefronts in two sets and the 64x64 tile 16 in four, the sets sharing each
// depth slice.
// Whether the direct-to-LDS loaders' 32-bit byte offsets hold a bm x kt slice of A and a bn x kt
// slice of B: every element of a slice lies below 2^30 bytes from its first (A(m, k) at
// a + m a_rs + k a_cs, B(k, n) at b + k b_rs + n b_cs; a K-major operand's lines are its rows, an
// M/N-major one's its depths, so deep slices of an M/N-major operand span kt - 1 line strides).
template <bool AK, bool BK>
bool direct_slices_fit(const GemmParams& p, int64_t bm, int64_t bn, int64_t kt) {
    const auto extent = [kt](bool kmaj, int64_t rows, int64_t line) {
        return kmaj ? (rows - 1) * line + kt : (kt - 1) * line + rows;
    };
    const int64_t a_line = AK ? p.a_rs : p.a_cs;
    const int64_t b_line = BK ? p.b_cs : p.b_rs;
    constexpr int64_t kLimit = int64_t{1} << 28; // floats
    return a_line >= 0 && b_line >= 0 && a_line < kLimit && b_line < kLimit &&
           extent(AK, bm, a_line) < kLimit && extent(BK, bn, b_line) < kLimit;
}

template <bool AK, bool BK>
void launch_layout(int tile, const GemmParams& p, int va, int vb, unsigned blocks, bool one_per_cu,
                   hipStream_t stream) {
    // With one workgroup per CU, no split and 16-byte operands, the 64x64 and 128x128 tiles run
    // the direct-to-LDS kernel (one accumulation chain, the tile kernels' depth order) in place of
    // the wavefront sets, on slices as deep as the CU's LDS allows (128 and 64: 138-148 KiB), so
    // each slice's MFMA work covers the next slice's load: 1024^3 28.9-29.5 -> 25.1-25.4 us,
    // 2048^3 146.2-152.2 -> 135.7-138.3 us across the four layouts.
    const auto direct_mid = [&](int64_t bm, int64_t bn, int64_t kt) {
        return one_per_cu && p.splits == 1 && va == 4 && vb == 4 &&
               direct_slices_fit<AK, BK>(p, bm, bn, kt);
    };
    switch (tile) {
    case MFR_TILE_256x256:
        // The direct-to-LDS form for every load width: with 16-byte operands it also beats the
        // register copy (4096^3 NT 1039 against 1075 us, 4096x4096x1024 286 against 300 us, the
        // same bits).
        if (va == 4 && vb == 4) {
            sgemm_direct_kernel<256, 256, 32, 4, 4, AK, BK, 4, 4><<<blocks, 1024, 0, stream>>>(p);
        } else if (va == 4) {
            sgemm_direct_kernel<256, 256, 32, 4, 4, AK, BK, 4, 1><<<blocks, 1024, 0, stream>>>(p);
        } else if (vb == 4) {
            sgemm_direct_kernel<256, 256, 32, 4, 4, AK, BK, 1, 4><<<blocks, 1024, 0, stream>>>(p);
        } else {
            sgemm_direct_kernel<256, 256, 32, 4, 4, AK, BK, 1, 1><<<blocks, 1024, 0, stream>>>(p);
        }
        break;
    case MFR_TILE_128x64:
        launch_vec<128, 64, 16, 2, 2, AK, BK>(p, va, vb, blocks, stream);
        break;
    case MFR_TILE_64x128:
        launch_vec<64, 128, 16, 2, 2, AK, BK>(p, va, vb, blocks, stream);
        break;
    case MFR_TILE_64x64:
        if (direct_mid(64, 64, 128)) {
            sgemm_direct_kernel<64, 64, 128, 2, 2, AK, BK, 4, 4><<<blocks, 256, 0, stream>>>(p);
        } else if (one_per_cu && p.splits == 1) {
            // 16 wavefronts: four sets of 2x2 share each 64-deep slice (4 per SIMD). 1024^3:
            // 31.0 -> 27.7 us; 16384 x 4 x 4096: 113.7 -> 94.2 us. Split depth ranges are
            // short and keep the 4-wavefront form (512^3 in two: 14.5 against 14.1 us).
            launch_vec<64, 64, 64, 2, 2, AK, BK, 4>(p, va, vb, blocks, stream);
        } else {
            launch_vec<64, 64, 32, 2, 2, AK, BK>(p, va, vb, blocks, stream);
        }
        break;
    default:
        if (direct_mid(128, 128, 64)) {
            sgemm_direct_kernel<128, 128, 64, 4, 4, AK, BK, 4, 4><<<blocks, 1024, 0, stream>>>(p);
        } else if (one_per_cu && p.splits == 1) {
            // 16 wavefronts: two sets of 2x4 share each 64-deep slice (4 per SIMD). 2048^3:
            // 150.2 -> 145.6 us; 2048 x 2048 x 8192: 583.9 -> 560.9 us (32-deep slices: 149.3
            // and 574.1 us).
            launch_vec<128, 128, 64, 2, 4, AK, BK, 2>(p, va, vb, blocks, stream);
        } else if (one_per_cu) {
            launch_vec<128, 128, 32, 2, 4, AK, BK>(p, va, vb, blocks, stream);
        } else {
            launch_vec<128, 128, 32, 2, 2, AK, BK>(p, va, vb, blocks, stream);
        }
        break;
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

// ---- operand staging --------------------------------------------------------------------------

// Batch dimensions of an operand that are not broadcast (nonzero stride), outermost first.
struct StageBatch {
    int dims;
    int64_t size[MFR_MAX_BATCH_DIMS];
    int64_t stride[MFR_MAX_BATCH_DIMS];
};

// dst line r (r = matrix * lines + line, matrices in the order of StageBatch) gets the `inner`
// unit-stride floats of source line `line` of that matrix, then zeros up to `pitch` (a multiple
// of 4); dst is 16-byte aligned and matrix-contiguous. One workgroup per line.
__global__ __launch_bounds__(256) void stage_kernel(const float* src, float* dst, int64_t lines,
                                                    int64_t inner, int64_t line_stride,
                                                    int64_t pitch, StageBatch sb) {
    const int64_t r = blockIdx.x;
    int64_t matrix = r / lines;
    const int64_t line = r - matrix * lines;
    int64_t offset = line * line_stride;
    for (int d = sb.dims - 1; d >= 0; --d) {
        const int64_t idx = matrix % sb.size[d];
        matrix /= sb.size[d];
        offset += idx * sb.stride[d];
    }
    const float* in = src + offset;
    float4* out = reinterpret_cast<float4*>(dst + r * pitch);
    for (int64_t u = threadIdx.x; u < pitch / 4; u += blockDim.x) {
        const int64_t c = 4 * u;
        float4 v;
        v.x = c < inner ? in[c] : 0.0f;
        v.y = c + 1 < inner ? in[c + 1] : 0.0f;
        v.z = c + 2 < inner ? in[c + 2] : 0.0f;
        v.w = c + 3 < inner ? in[c + 3] : 0.0f;
        out[u] = v;
    }
}

// One operand as the loader reads it: `lines` lines of `inner` unit-stride floats, `line_stride`
// apart (the stride of its other matrix dimension), plus its batch strides. For A that is
// (m lines of k) when K-major, else (k lines of m); for B (n lines of k) or (k lines of n).
struct Operand {
    const float* base;
    int64_t lines, inner;
    int64_t* line_stride; // the GemmParams field holding it, rewritten when staged
    int64_t* unit_stride; // the GemmParams field holding the unit stride
    int64_t* batch_stride;
};

int64_t round4(int64_t v) { return (v + 3) / 4 * 4; }

// Floats of the staged copy of `o` under batch shape p.batch (broadcast dimensions once).
int64_t staged_floats(const Operand& o, const GemmParams& p) {
    int64_t count = o.lines * round4(o.inner);
    for (int d = 0; d < p.batch_dims; ++d) {
        if (o.batch_stride[d] != 0) {
            count *= p.batch[d];
        }
    }
    return count;
}

void repoint_staged(Operand& o, float* dst, const GemmParams& p);

// Copies `o` into dst (staged_floats(o, p) floats, 16-byte aligned) and points the GEMM at it.
void stage_operand(Operand& o, float* dst, const GemmParams& p, hipStream_t stream) {
    const int64_t pitch = round4(o.inner);
    StageBatch sb{};
    int64_t matrices = 1;
    for (int d = 0; d < p.batch_dims; ++d) {
        if (o.batch_stride[d] != 0) {
            sb.size[sb.dims] = p.batch[d];
            sb.stride[sb.dims] = o.batch_stride[d];
            ++sb.dims;
            matrices *= p.batch[d];
        }
    }
    const int64_t rows = matrices * o.lines;
    mfr::require(rows < (int64_t{1} << 31), "sgemm: operand too large to stage");
    stage_kernel<<<static_cast<unsigned>(rows), 256, 0, stream>>>(o.base, dst, o.lines, o.inner,
                                                                  *o.line_stride, pitch, sb);
    mfr::check_launch("stage_kernel");
    repoint_staged(o, dst, p);
}

// Points the GEMM at o's staged copy in dst: lines round4(inner) apart, matrices contiguous in
// the order of StageBatch.
void repoint_staged(Operand& o, float* dst, const GemmParams& p) {
    const int64_t pitch = round4(o.inner);
    int64_t next = o.lines * pitch;
    for (int d = p.batch_dims - 1; d >= 0; --d) {
        if (o.batch_stride[d] != 0) {
            o.batch_stride[d] = next;
            next *= p.batch[d];
        }
    }
    *o.line_stride = pitch;
    *o.unit_stride = 1;
    o.base = dst;
}

// Workspace of `bytes`, or nullptr when it cannot be had (the failed allocation's error is
// cleared so the next launch check does not report it).
void* try_reserve(mfr_stream& s, size_t bytes) {
    try {
        return s.reserve(bytes);
    } catch (const mfr::Error&) {
        (void)hipGetLastError();
        return nullptr;
    }
}

// Everything mfr_sgemm decides before launching: the kernel parameters (strides of extent-1
// dimensions normalised), each operand's layout and load width, which operands to stage, and the
// tile. mfr_sgemm_plan reports it without launching.
// A rectangle of the output run as one launch (plus its reduce when split).
struct Region {
    int64_t m_off = 0, n_off = 0, m = 0, n = 0;
    int tile = MFR_TILE_AUTO;
    int splits = 1;  // depth ranges (split-K when > 1)
    int64_t per = 0; // depth of each range
};

struct Plan {
    GemmParams p{};
    bool empty = false;        // nothing to compute (m, n or the batch is 0)
    bool ak = true, bk = true; // K-major operands
    int va = 4, vb = 4;        // load widths read in place
    bool stage_a = false, stage_b = false;
    bool c0 = false;           // beta * C0 is read
    Region regions[4];         // [0] is the main one; the rest are peeled edge strips
    int region_count = 1;
};

// m x n: the output rectangle the thin path would take (the product or an edge strip, whose
// offset is a multiple of a tile and keeps the alignment).
int thin_b_layout(const GemmParams& p, const Plan& plan, int64_t m, int64_t n) {
    bool along_n = true;
    if (!thin_possible(m, n, plan.ak, plan.bk, &along_n)) {
        return 0;
    }
    if (along_n ? plan.stage_b : plan.stage_a) {
        return 2;
    }
    const float* base = along_n ? p.b : p.a;
    const int64_t unit = along_n ? p.b_cs : p.a_rs;
    const int64_t line = along_n ? p.b_rs : p.a_cs;
    const int64_t* batch_strides = along_n ? p.b_bs : p.a_bs;
    bool aligned = unit == 1 && line % 4 == 0 && reinterpret_cast<uintptr_t>(base) % 16 == 0;
    for (int d = 0; d < p.batch_dims; ++d) {
        aligned = aligned && batch_strides[d] % 4 == 0;
    }
    return aligned ? 1 : 0;
}

// The plan's output as one region with `choice`.
void single_region(Plan& plan, const Choice& choice) {
    plan.region_count = 1;
    plan.regions[0] = Region{0, 0, plan.p.m, plan.p.n, choice.tile, choice.splits, choice.per};
}

// ---- edge peeling ----------------------------------------------------------------------------
//
// A dimension a few rows past a multiple of a big tile (N = 4099 = 16 x 256 + 3) costs that tile a
// whole extra wave of tiles for a sliver of work. In AUTO, such a remainder (at most a quarter of
// the tile) may be peeled off: the main rectangle runs on the big tile, and each edge strip runs
// as a launch of its own, with its own tile and split count. The peeled plan is kept when the
// model prices it (plus kLaunchUs per extra launch) at least 5% below the best single launch.
constexpr double kLaunchUs = 5.0;
constexpr double kPeelMargin = 0.95;

bool big_tile_ok(const Plan& plan);

void consider_peeling(Plan& plan, int64_t batch, int cus, double single_us) {
    const GemmParams& p = plan.p;
    double best_us = single_us * kPeelMargin;
    for (int t = 1; t < MFR_TILE_THIN; ++t) {
        const int64_t bm = kTiles[t].bm, bn = kTiles[t].bn;
        const int64_t rem_m = p.m % bm, rem_n = p.n % bn;
        const bool peel_m = p.m > bm && rem_m > 0 && rem_m * 4 <= bm;
        const bool peel_n = p.n > bn && rem_n > 0 && rem_n * 4 <= bn;
        if (!peel_m && !peel_n) {
            continue;
        }
        const int64_t main_m = peel_m ? p.m - rem_m : p.m;
        const int64_t main_n = peel_n ? p.n - rem_n : p.n;
        Region regions[4];
        int count = 0;
        const Choice main =
            choose(main_m, main_n, p.k, batch, cus, t, 1, plan.c0, plan.ak, plan.bk,
                   thin_b_layout(p, plan, main_m, main_n), big_tile_ok(plan));
        regions[count++] = Region{0, 0, main_m, main_n, main.tile, main.splits, main.per};
        double us = main.us;
        auto strip = [&](int64_t m_off, int64_t n_off, int64_t m, int64_t n) {
            const Choice c =
                choose(m, n, p.k, batch, cus, MFR_TILE_AUTO, 0, plan.c0, plan.ak, plan.bk,
                       thin_b_layout(p, plan, m, n), big_tile_ok(plan));
            regions[count++] = Region{m_off, n_off, m, n, c.tile, c.splits, c.per};
            us += c.us + kLaunchUs;
        };
        if (peel_n) {
            strip(0, main_n, main_m, rem_n);
        }
        if (peel_m) {
            strip(main_m, 0, rem_m, main_n);
        }
        if (peel_m && peel_n) {
            strip(main_m, main_n, rem_m, rem_n);
        }
        if (us < best_us) {
            best_us = us;
            plan.region_count = count;
            for (int i = 0; i < count; ++i) {
                plan.regions[i] = regions[i];
            }
        }
    }
}

Operand operand_a(GemmParams& p, bool ak) {
    return Operand{p.a, ak ? p.m : p.k, ak ? p.k : p.m, ak ? &p.a_rs : &p.a_cs,
                   ak ? &p.a_cs : &p.a_rs, p.a_bs};
}

Operand operand_b(GemmParams& p, bool bk) {
    return Operand{p.b, bk ? p.n : p.k, bk ? p.k : p.n, bk ? &p.b_cs : &p.b_rs,
                   bk ? &p.b_rs : &p.b_cs, p.b_bs};
}

int64_t staged_floats_padded(const Operand& o, const GemmParams& p) {
    return (staged_floats(o, p) + 63) / 64 * 64; // 256-byte aligned parts of the workspace
}

// Whether the 256x256 tile can read the plan's operands (as they will be after staging): it
// copies both slices straight into LDS with buffer loads, whose byte offsets within a slice must
// stay below 2^30: 255 lines of a K-major operand, or 31 depth lines of the other, plus a line's
// own extent.
bool big_tile_ok(const Plan& plan) {
    GemmParams p = plan.p;
    const auto fits = [](const Operand& o, bool kmaj, bool staged) {
        const int64_t line = staged ? round4(o.inner) : *o.line_stride;
        const int64_t last = kmaj ? 255 * line + 32 : 31 * line + 256;
        return line >= 0 && last < (int64_t{1} << 28);
    };
    return fits(operand_a(p, plan.ak), plan.ak, plan.stage_a) &&
           fits(operand_b(p, plan.bk), plan.bk, plan.stage_b);
}

// Whether the panel path (panel_kernel.hpp) can take the plan's product: a depth of 1 to 64, both
// operands read along k with 16-byte loads in place, no activation, and every byte offset its
// buffer resources use (within a batch matrix) below 2^31.
bool panel_fits(const Plan& plan) {
    const GemmParams& p = plan.p;
    if (!plan.ak || !plan.bk || plan.va != 4 || plan.vb != 4 || plan.stage_a || plan.stage_b) {
        return false;
    }
    if (p.k < 1 || p.k > kPanelMaxDepth || p.act != MFR_ACT_NONE) {
        return false;
    }
    const double limit = 2147483648.0;
    const double m = static_cast<double>(p.m);
    return (m + 32.0) * p.c_rs * 4.0 < limit && (!plan.c0 || (m + 32.0) * p.c0_rs * 4.0 < limit) &&
           m * p.a_rs * 4.0 + 4.0 * p.k < limit && (kPanelCols + 1.0) * p.b_cs * 4.0 < limit;
}

// AUTO takes the panel path for products it fits with more than one panel of rows and at least
// 16 MiB of output, where the tile kernels pay their store time on top of their MFMA time.
bool panel_preferred(const Plan& plan) {
    const GemmParams& p = plan.p;
    return panel_fits(plan) && p.m > kPanelRows / 2 &&
           static_cast<double>(p.m) * p.n * p.batch_count >= 4194304.0;
}

// Validates d (the checks and error codes of mfr_sgemm) and makes the plan for a device with
// `cus` compute units.
Plan plan_sgemm(const mfr_gemm_desc& d, int cus) {
    using mfr::require;
    require(d.m >= 0 && d.n >= 0 && d.k >= 0, "sgemm: negative dimension");
    require(d.batch_dims >= 0 && d.batch_dims <= MFR_MAX_BATCH_DIMS,
            "sgemm: batch_dims out of range");
    require(d.act == MFR_ACT_NONE || d.act == MFR_ACT_GELU_TANH || d.act == MFR_ACT_GELU_ERF,
            "sgemm: unknown activation");
    require(d.tile >= MFR_TILE_AUTO && d.tile < MFR_TILE_COUNT, "sgemm: unknown tile");
    require(d.stage == MFR_STAGE_AUTO || d.stage == MFR_STAGE_NEVER || d.stage == MFR_STAGE_ALWAYS,
            "sgemm: unknown stage mode");
    require(d.splits >= 0 && d.splits <= kMaxSplits, "sgemm: splits out of range");
    require(d.flags == 0 || d.flags == MFR_GEMM_CAUSAL, "sgemm: unknown flags");
    Plan plan;
    GemmParams& p = plan.p;
    int64_t batch_count = 1;
    for (int i = 0; i < d.batch_dims; ++i) {
        require(d.batch[i] >= 0, "sgemm: negative batch size");
        batch_count *= d.batch[i];
    }
    if (d.m == 0 || d.n == 0 || batch_count == 0) {
        plan.empty = true;
        return plan;
    }
    require(d.c != nullptr, "sgemm: null c");
    require(d.m == 1 || d.c_rs >= d.n, "sgemm: c row stride smaller than n");
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
    p.causal = d.flags == MFR_GEMM_CAUSAL ? 1 : 0;
    if (p.beta != 0.0f && p.c0 != nullptr) {
        require(p.m == 1 || p.c0_rs >= p.n, "sgemm: c0 row stride smaller than n");
    }

    // A dimension of extent 1 is never stepped along, so its stride is free: pick the one that
    // gives the operand a unit stride. With k == 0 nothing is loaded at all.
    if (d.k > 0) {
        require(d.a != nullptr && d.b != nullptr, "sgemm: null a or b");
        if (p.k == 1 && p.a_cs != 1) p.a_cs = 1;
        if (p.m == 1 && p.a_cs != 1) p.a_rs = 1;
        if (p.k == 1 && p.b_rs != 1 && p.b_cs != 1) p.b_rs = 1;
        if (p.n == 1 && p.b_rs != 1) p.b_cs = 1;
        if (p.a_cs == 1) {
            plan.ak = true;
        } else if (p.a_rs == 1) {
            plan.ak = false;
        } else {
            throw mfr::Error(MFR_E_UNSUPPORTED, "sgemm: A needs a unit stride along a dimension");
        }
        if (p.b_rs == 1) {
            plan.bk = true;
        } else if (p.b_cs == 1) {
            plan.bk = false;
        } else {
            throw mfr::Error(MFR_E_UNSUPPORTED, "sgemm: B needs a unit stride along a dimension");
        }
        plan.va = plan.ak ? vector_width(p.a, p.k, p.a_rs, p.m, p.a_bs, p.batch_dims)
                          : vector_width(p.a, p.m, p.a_cs, p.k, p.a_bs, p.batch_dims);
        plan.vb = plan.bk ? vector_width(p.b, p.k, p.b_cs, p.n, p.b_bs, p.batch_dims)
                          : vector_width(p.b, p.n, p.b_rs, p.k, p.b_bs, p.batch_dims);
    }

    // Staging (see the design notes at the top): ALWAYS, or AUTO when the product is large next
    // to the copy.
    if ((plan.va == 1 || plan.vb == 1) && d.stage != MFR_STAGE_NEVER) {
        const Operand oa = operand_a(p, plan.ak);
        const Operand ob = operand_b(p, plan.bk);
        const int64_t fa = plan.va == 1 ? staged_floats_padded(oa, p) : 0;
        const int64_t fb = plan.vb == 1 ? staged_floats_padded(ob, p) : 0;
        const double flops = 2.0 * static_cast<double>(p.m) * p.n * p.k * batch_count;
        const double staged_bytes = 4.0 * static_cast<double>(fa + fb);
        const bool worth = flops >= 1073741824.0 && staged_bytes * 64.0 <= flops &&
                           staged_bytes <= 4294967296.0;
        if (d.stage == MFR_STAGE_ALWAYS || worth) {
            plan.stage_a = plan.va == 1;
            plan.stage_b = plan.vb == 1;
        }
    }
    plan.c0 = p.c0 != nullptr && p.beta != 0.0f;
    const auto tile_plan = [&](Plan& q) {
        if (p.causal != 0 && !(d.tile == MFR_TILE_PANEL || d.tile == MFR_TILE_AUTO)) {
            throw mfr::Error(MFR_E_UNSUPPORTED,
                             "sgemm: the causal mask is taken by the panel path only");
        }
        if (d.tile == MFR_TILE_PANEL || p.causal != 0 ||
            (d.tile == MFR_TILE_AUTO && d.splits <= 1 && panel_preferred(q))) {
            if (!panel_fits(q) || d.splits > 1) {
                throw mfr::Error(MFR_E_UNSUPPORTED,
                                 "sgemm: the panel path takes k <= 64 with both operands read "
                                 "along k by 16-byte loads in place, no activation and no split");
            }
            single_region(q, Choice{MFR_TILE_PANEL, 1, p.k, 0.0});
            return;
        }
        const Choice choice = choose(p.m, p.n, p.k, batch_count, cus, d.tile, d.splits, q.c0,
                                     q.ak, q.bk, thin_b_layout(q.p, q, p.m, p.n), big_tile_ok(q));
        single_region(q, choice);
        if (d.tile == MFR_TILE_AUTO && d.splits == 0) {
            consider_peeling(q, batch_count, cus, choice.us);
        }
    };
    tile_plan(plan);
    // AUTO staging under the 256x256 tile: an operand whose unit stride runs along its rows (M
    // or N) is read in place instead. Its direct-to-LDS slices are whole runs of 256 floats,
    // about one cache line more per run than the aligned copy, where a K-major operand's runs of
    // 32 floats would touch twice the lines. configs[3]: X staged and W in place 323 us, both
    // staged 331 us, both in place 333 us.
    if (d.stage == MFR_STAGE_AUTO && plan.regions[0].tile == MFR_TILE_256x256 &&
        ((plan.stage_a && !plan.ak) || (plan.stage_b && !plan.bk))) {
        Plan partial = plan;
        partial.stage_a = plan.stage_a && plan.ak;
        partial.stage_b = plan.stage_b && plan.bk;
        if (big_tile_ok(partial)) {
            tile_plan(partial);
            if (partial.regions[0].tile == MFR_TILE_256x256) {
                plan = partial;
            }
        }
    }
    for (int i = 0; i < plan.region_count; ++i) {
        const Region& r = plan.regions[i];
        require(r.splits <= 1 ||
                    4.0 * r.splits * static_cast<double>(r.m) * r.n * batch_count <= 17179869184.0,
                "sgemm: split-K partial sums over 16 GiB");
    }
    return plan;
}

// Floats of workspace for the split-K partial sums of `plan` (256-byte aligned): the largest any
// region needs, since regions run one after another on the stream.
int64_t partial_floats(const Plan& plan) {
    int64_t most = 0;
    for (int i = 0; i < plan.region_count; ++i) {
        const Region& r = plan.regions[i];
        if (r.splits > 1) {
            const int64_t f = (r.splits * r.m * r.n * plan.p.batch_count + 63) / 64 * 64;
            most = f > most ? f : most;
        }
    }
    return most;
}

// The thin path on the product q describes (thin_possible holds): C = A B by rows of A when
// n <= 8 and A is read along k, else C^T = B^T A^T by rows of B^T. With stage != nullptr (rows of
// A read 4 bytes at a time, one matrix, k * columns within kStripLdsFloats), the same launch also
// writes A's zero-padded copy, lines stage_rs floats apart (strip_stage_kernel).
void launch_thin(const Plan& plan, const GemmParams& q, int va, int vb, hipStream_t stream,
                 float* stage = nullptr, int64_t stage_rs = 0) {
    ThinParams t{};
    bool along_n = true;
    thin_possible(q.m, q.n, plan.ak, plan.bk, &along_n);
    const float* c0 = q.c0 != nullptr && q.beta != 0.0f ? q.c0 : nullptr;
    const int64_t* a_bs = q.a_bs;
    const int64_t* b_bs = q.b_bs;
    int width = va;
    if (along_n) {
        t.a = q.a;
        t.a_rs = q.a_rs;
        t.a_cs = q.a_cs;
        t.b = q.b;
        t.b_rs = q.b_rs;
        t.b_cs = q.b_cs;
        t.rows = q.m;
        t.cols = q.n;
        t.c_rs = q.c_rs;
        t.c_cs = 1;
        t.c0_rs = q.c0_rs;
        t.c0_cs = 1;
        t.bias_rs = 0;
        t.bias_cs = 1;
    } else {
        // A'(j, p) = B(p, j), B'(p, i) = A(i, p), C'(j, i) = C(i, j), bias'(j, i) = bias[j].
        t.a = q.b;
        t.a_rs = q.b_cs;
        t.a_cs = q.b_rs;
        t.b = q.a;
        t.b_rs = q.a_cs;
        t.b_cs = q.a_rs;
        t.rows = q.n;
        t.cols = q.m;
        t.c_rs = 1;
        t.c_cs = q.c_rs;
        t.c0_rs = 1;
        t.c0_cs = q.c0_rs;
        t.bias_rs = 1;
        t.bias_cs = 0;
        a_bs = q.b_bs;
        b_bs = q.a_bs;
        width = vb;
    }
    t.c = q.c;
    t.c0 = c0;
    t.bias = q.bias;
    t.k = q.k;
    t.batch_dims = q.batch_dims;
    for (int d = 0; d < q.batch_dims; ++d) {
        t.batch[d] = q.batch[d];
        t.a_bs[d] = a_bs[d];
        t.b_bs[d] = b_bs[d];
        t.c_bs[d] = q.c_bs[d];
        t.c0_bs[d] = q.c0_bs[d];
    }
    t.act = q.act;
    t.alpha = q.alpha;
    t.beta = q.beta;
    t.blocks_per_batch = (t.rows + kThinDotRows - 1) / kThinDotRows;
    t.stage = stage;
    t.stage_rs = stage_rs;
    mfr::require(stage == nullptr || (along_n && width == 1 && q.batch_count == 1),
                 "sgemm: the strip stages A only from 4-byte rows of one matrix");
    const int64_t blocks = t.blocks_per_batch * q.batch_count;
    mfr::require(blocks < (int64_t{1} << 31), "sgemm: problem too large for one launch");
    const unsigned grid = static_cast<unsigned>(blocks);
    // The column count rounded up to 1, 2, 4 or 8 (kThinCols).
    const int c = t.cols <= 1 ? 1 : t.cols <= 2 ? 2 : t.cols <= 4 ? 4 : kThinCols;
    // B' pieces of 2 or 4 floats: unit column stride, rows and batches aligned to the piece, and
    // the c columns in memory (exactly c, or a staged B' whose lines are zero-padded to a
    // multiple of 4).
    const bool b_padded = along_n ? plan.stage_b : plan.stage_a;
    const int piece = c == 2 ? 2 : 4;
    bool b_pieces = c >= 2 && t.b_cs == 1 && t.b_rs % piece == 0 &&
                    reinterpret_cast<uintptr_t>(t.b) % (4 * piece) == 0 &&
                    (t.cols == c || b_padded);
    for (int d = 0; d < t.batch_dims; ++d) {
        b_pieces = b_pieces && t.b_bs[d] % piece == 0;
    }
    if (stage != nullptr) {
        mfr::require(t.k * c <= kStripLdsFloats, "sgemm: the strip's B' does not fit in LDS");
        const unsigned strip_grid = static_cast<unsigned>((t.rows + kStripWaves - 1) / kStripWaves);
        const size_t lds = sizeof(float) * static_cast<size_t>(t.k * c);
        switch (c) {
        case 1: strip_stage_kernel<1><<<strip_grid, 64 * kStripWaves, lds, stream>>>(t); break;
        case 2: strip_stage_kernel<2><<<strip_grid, 64 * kStripWaves, lds, stream>>>(t); break;
        case 4: strip_stage_kernel<4><<<strip_grid, 64 * kStripWaves, lds, stream>>>(t); break;
        default:
            strip_stage_kernel<kThinCols><<<strip_grid, 64 * kStripWaves, lds, stream>>>(t);
        }
        mfr::check_launch("strip_stage_kernel");
        return;
    }
    if (b_pieces) {
        if (width == 4) {
            switch (c) {
            case 2: thin_dot_kernel<4, 2, true><<<grid, kThinThreads, 0, stream>>>(t); break;
            case 4: thin_dot_kernel<4, 4, true><<<grid, kThinThreads, 0, stream>>>(t); break;
            default:
                if (t.rows >= kThinLdsMinRows) {
                    // B' staged in LDS: 16 rows per workgroup.
                    constexpr int rows = thin_lds_rows<kThinLdsWaves>();
                    t.blocks_per_batch = (t.rows + rows - 1) / rows;
                    const unsigned lds_grid =
                        static_cast<unsigned>(t.blocks_per_batch * q.batch_count);
                    thin_dot_lds_kernel<kThinLdsWaves>
                        <<<lds_grid, 64 * kThinLdsWaves, 0, stream>>>(t);
                } else {
                    thin_dot_kernel<4, kThinCols, true><<<grid, kThinThreads, 0, stream>>>(t);
                }
            }
        } else {
            switch (c) {
            case 2: thin_dot_kernel<1, 2, true><<<grid, kThinThreads, 0, stream>>>(t); break;
            case 4: thin_dot_kernel<1, 4, true><<<grid, kThinThreads, 0, stream>>>(t); break;
            default: thin_dot_kernel<1, kThinCols, true><<<grid, kThinThreads, 0, stream>>>(t);
            }
        }
        mfr::check_launch("thin_dot_kernel");
        return;
    }
    if (width == 4) {
        switch (c) {
        case 1: thin_dot_kernel<4, 1><<<grid, kThinThreads, 0, stream>>>(t); break;
        case 2: thin_dot_kernel<4, 2><<<grid, kThinThreads, 0, stream>>>(t); break;
        case 4: thin_dot_kernel<4, 4><<<grid, kThinThreads, 0, stream>>>(t); break;
        default: thin_dot_kernel<4, kThinCols><<<grid, kThinThreads, 0, stream>>>(t); break;
        }
    } else {
        switch (c) {
        case 1: thin_dot_kernel<1, 1><<<grid, kThinThreads, 0, stream>>>(t); break;
        case 2: thin_dot_kernel<1, 2><<<grid, kThinThreads, 0, stream>>>(t); break;
        case 4: thin_dot_kernel<1, 4><<<grid, kThinThreads, 0, stream>>>(t); break;
        default: thin_dot_kernel<1, kThinCols><<<grid, kThinThreads, 0, stream>>>(t); break;
        }
    }
    mfr::check_launch("thin_dot_kernel");
}

// Whether the epilogue writes q's C with non-temporal stores: the output is larger than the
// last-level cache (256 MiB of Infinity Cache), so no later kernel finds it there anyway, and
// every row starts on a 128-byte line, so the streamed writes are whole lines. The composed
// attention's scores (128 x 1024 x 1024, 512 MiB): 223.8 -> 201 us. Rows off the lines are
// slower streamed (the MLP's 4099-float rows, whose tile edges write partial lines: 321.5 ->
// 334.5 us); 4096^3 and 2048^3 are unchanged either way.
bool streamed_output(const GemmParams& q) {
    if (4.0 * static_cast<double>(q.m) * q.n * q.batch_count <= mfr::kLastLevelCacheBytes) {
        return false;
    }
    if (reinterpret_cast<uintptr_t>(q.c) % 128 != 0 || q.c_rs % 32 != 0) {
        return false;
    }
    for (int d = 0; d < q.batch_dims; ++d) {
        if (q.c_bs[d] % 32 != 0) {
            return false;
        }
    }
    return true;
}

// Whether the 128x64 tile runs as sgemm_pair_kernel on q: A read along k and B along n, both by
// 16-byte loads, one tile of columns (n <= 64), and each slice's byte offsets below 2^30 (the
// direct-to-LDS loaders' 32-bit offsets, as big_tile_ok).
bool pair_fits(const Plan& plan, const GemmParams& q, int va, int vb) {
    return plan.ak && !plan.bk && va == 4 && vb == 4 && q.n <= 64 &&
           127.0 * q.a_rs + 32.0 < 268435456.0 && 31.0 * q.b_rs + 64.0 < 268435456.0;
}

// Launches the kernel (and the reduce, when split) for region r of the product p describes.
void launch_region(const Plan& plan, const GemmParams& p, const Region& r, int va, int vb,
                   float* partial, int cus, hipStream_t stream, float* stage = nullptr,
                   int64_t stage_rs = 0) {
    using mfr::require;
    GemmParams q = p;
    q.m = r.m;
    q.n = r.n;
    q.a = p.a + r.m_off * p.a_rs;
    q.b = p.b + r.n_off * p.b_cs;
    q.c = p.c + r.m_off * p.c_rs + r.n_off;
    q.c0 = p.c0 != nullptr ? p.c0 + r.m_off * p.c0_rs + r.n_off : nullptr;
    q.bias = p.bias != nullptr ? p.bias + r.n_off : nullptr;
    if (r.tile == MFR_TILE_THIN) {
        launch_thin(plan, q, va, vb, stream, stage, stage_rs);
        return;
    }
    if (r.tile == MFR_TILE_PANEL) {
        launch_panel(q, streamed_output(q), cus, stream);
        mfr::check_launch("sgemm_panel_kernel");
        return;
    }
    const int tile = r.tile;
    const int64_t tiles_m = (q.m + kTiles[tile].bm - 1) / kTiles[tile].bm;
    const int64_t tiles_n = (q.n + kTiles[tile].bn - 1) / kTiles[tile].bn;
    const int64_t blocks = tiles_m * tiles_n * q.batch_count * r.splits;
    require(tiles_m < (int64_t{1} << 30) && tiles_n < (int64_t{1} << 30) &&
                blocks < (int64_t{1} << 31),
            "sgemm: problem too large for one launch");
    q.tiles_m = static_cast<int32_t>(tiles_m);
    q.tiles_n = static_cast<int32_t>(tiles_n);
    q.group_m = kGroupM;
    q.splits = r.splits;
    q.k_per_split = r.splits > 1 ? r.per : q.k;
    q.partial = r.splits > 1 ? partial : nullptr;
    q.stream_c = q.partial == nullptr && streamed_output(q) ? 1 : 0;
    const unsigned grid = static_cast<unsigned>(blocks);
    const bool one_per_cu = blocks <= cus;
    if (tile == MFR_TILE_128x64 && pair_fits(plan, q, va, vb)) {
        sgemm_pair_kernel<32><<<grid, 256, 0, stream>>>(q);
    } else if (plan.ak && plan.bk) {
        launch_layout<true, true>(tile, q, va, vb, grid, one_per_cu, stream);
    } else if (plan.ak) {
        launch_layout<true, false>(tile, q, va, vb, grid, one_per_cu, stream);
    } else if (plan.bk) {
        launch_layout<false, true>(tile, q, va, vb, grid, one_per_cu, stream);
    } else {
        launch_layout<false, false>(tile, q, va, vb, grid, one_per_cu, stream);
    }
    mfr::check_launch("sgemm_kernel");
    if (q.partial != nullptr) {
        const int64_t lines = q.m * q.batch_count;
        const dim3 reduce_grid(mfr::grid_blocks(q.n, 256, 64),
                               static_cast<unsigned>(lines < 65535 ? lines : 65535));
        split_reduce_kernel<<<reduce_grid, 256, 0, stream>>>(q);
        mfr::check_launch("split_reduce_kernel");
    }
}

// ---- plan cache ---------------------------------------------------------------------------------

// Planning (the tile and split model, edge peeling) costs 0.2-1.1 us of host time per call, next to
// about 3 us per kernel launch (a C++ caller submitting 300 x 260 x 516 with two splits: 7.2 ->
// 6.2 us per call with the cache; 64^3: 3.17 -> 3.02 us). A plan is a function of the descriptor's
// shapes, strides and
// settings, of which pointers are null, the 16-byte alignment of a and b, whether beta is 0, and
// the device's CU count (alpha, beta's value, the bias pointer and the activation are only copied
// into it). Each thread keeps the plans it made in a small direct-mapped table under that key and
// reuses one with the call's own pointers and scalars.
struct PlanKey {
    int64_t v[40];
};

PlanKey plan_key(const mfr_gemm_desc& d, int cus) {
    PlanKey key{};
    int i = 0;
    auto put = [&](int64_t x) { key.v[i++] = x; };
    const int dims = d.batch_dims >= 0 && d.batch_dims <= MFR_MAX_BATCH_DIMS ? d.batch_dims : 0;
    put(d.m);
    put(d.n);
    put(d.k);
    put(d.batch_dims);
    put(d.act);
    put(d.a_rs);
    put(d.a_cs);
    put(d.b_rs);
    put(d.b_cs);
    put(d.c_rs);
    put(d.c0_rs);
    for (int j = 0; j < MFR_MAX_BATCH_DIMS; ++j) {
        const bool live = j < dims;
        put(live ? d.batch[j] : 0);
        put(live ? d.a_bs[j] : 0);
        put(live ? d.b_bs[j] : 0);
        put(live ? d.c_bs[j] : 0);
        put(live ? d.c0_bs[j] : 0);
    }
    put(d.tile);
    put(d.stage);
    put(d.splits);
    put(d.flags);
    put((d.a == nullptr ? 1 : 0) | (d.b == nullptr ? 2 : 0) | (d.c == nullptr ? 4 : 0) |
        (d.c0 == nullptr ? 8 : 0) | (d.beta != 0.0f ? 16 : 0) | (mfr::aligned16(d.a) ? 32 : 0) |
        (mfr::aligned16(d.b) ? 64 : 0));
    put(cus);
    return key;
}

constexpr int kPlanSlots = 32;

struct PlanSlot {
    bool valid = false;
    PlanKey key{};
    Plan plan;
};

// The plan for d (plan_sgemm's, which validates d; an invalid d is never cached).
Plan cached_plan(const mfr_gemm_desc& d, int cus) {
    static_assert(11 + 5 * MFR_MAX_BATCH_DIMS + 6 <= 40, "PlanKey holds every field");
    thread_local PlanSlot slots[kPlanSlots];
    const PlanKey key = plan_key(d, cus);
    uint64_t hash = 1469598103934665603ull; // FNV-1a over the key's words
    for (const int64_t x : key.v) {
        hash = (hash ^ static_cast<uint64_t>(x)) * 1099511628211ull;
    }
    PlanSlot& slot = slots[hash % kPlanSlots];
    if (slot.valid && std::memcmp(&slot.key, &key, sizeof(PlanKey)) == 0) {
        Plan plan = slot.plan;
        plan.p.a = d.a;
        plan.p.b = d.b;
        plan.p.c = d.c;
        plan.p.c0 = d.c0;
        plan.p.bias = d.bias;
        plan.p.alpha = d.alpha;
        plan.p.beta = d.beta;
        return plan;
    }
    Plan plan = plan_sgemm(d, cus);
    slot.key = key;
    slot.plan = plan;
    slot.valid = true;
    return plan;
}

// Runs d on s. The split-K partial sums and staged operands go to one workspace laid out
// [partial sums][staged A][staged B]: the stream's own (grown as needed, with fallbacks when it
// cannot be had), or, when `scratch` is not null, that fixed buffer of `scratch_bytes`, in which
// case a plan needing more is refused before anything is launched.
void run_sgemm(mfr_stream& s, const mfr_gemm_desc& d, float* scratch = nullptr,
               size_t scratch_bytes = 0) {
    Plan plan = cached_plan(d, s.compute_units);
    if (plan.empty) {
        return;
    }
    GemmParams& p = plan.p;
    int va = plan.va, vb = plan.vb;
    Operand oa = operand_a(p, plan.ak);
    Operand ob = operand_b(p, plan.bk);
    int64_t fa = plan.stage_a ? staged_floats_padded(oa, p) : 0;
    int64_t fb = plan.stage_b ? staged_floats_padded(ob, p) : 0;
    float* ws = nullptr;
    std::unique_lock<std::mutex> hold(s.workspace_mutex, std::defer_lock);
    if (scratch != nullptr) {
        // The fixed array instead of the stream's workspace. A plan that needs more than it holds
        // takes the fallbacks the workspace path takes when memory cannot be had, where the
        // caller left them open: automatic splits become one range, automatic staging reads the
        // operands in place. Anything still over the maximum is refused before any launch.
        const auto need = [&] { return 4 * static_cast<size_t>(partial_floats(plan) + fa + fb); };
        if (need() > scratch_bytes && partial_floats(plan) > 0 && d.splits == 0) {
            single_region(plan, choose(p.m, p.n, p.k, p.batch_count, s.compute_units, d.tile, 1,
                                       plan.c0, plan.ak, plan.bk,
                                       thin_b_layout(p, plan, p.m, p.n), big_tile_ok(plan)));
        }
        if (need() > scratch_bytes && fa + fb > 0 && d.stage == MFR_STAGE_AUTO) {
            plan.stage_a = plan.stage_b = false;
            fa = fb = 0;
            if (d.tile == MFR_TILE_AUTO) {
                single_region(plan, choose(p.m, p.n, p.k, p.batch_count, s.compute_units,
                                           MFR_TILE_AUTO, d.splits == 0 ? 1 : d.splits, plan.c0,
                                           plan.ak, plan.bk, thin_b_layout(p, plan, p.m, p.n),
                                           big_tile_ok(plan)));
            }
        }
        if (need() > scratch_bytes) {
            throw mfr::Error(MFR_E_INVALID,
                             "sgemm_noalloc: this product needs " + std::to_string(need()) +
                                 " bytes of scratch (split-K sums and staged operands), more "
                                 "than the " + std::to_string(scratch_bytes) + "-byte maximum");
        }
        ws = scratch;
    } else if (partial_floats(plan) + fa + fb > 0) {
        // Held until every launch is queued (see mfr_stream).
        hold.lock();
        ws = static_cast<float*>(
            try_reserve(s, 4 * static_cast<size_t>(partial_floats(plan) + fa + fb)));
        if (ws == nullptr && partial_floats(plan) > 0 && d.splits == 0) {
            // Automatic splits without the memory: one region, one range.
            single_region(plan, choose(p.m, p.n, p.k, p.batch_count, s.compute_units, d.tile, 1,
                                       plan.c0, plan.ak, plan.bk,
                                       thin_b_layout(p, plan, p.m, p.n), big_tile_ok(plan)));
            if (fa + fb > 0) {
                ws = static_cast<float*>(try_reserve(s, 4 * static_cast<size_t>(fa + fb)));
            }
        }
        if (ws == nullptr && partial_floats(plan) + fa + fb > 0) {
            if (partial_floats(plan) > 0) {
                throw mfr::Error(MFR_E_RUNTIME, "sgemm: no workspace for split-K partial sums");
            }
            if (d.stage == MFR_STAGE_ALWAYS) {
                throw mfr::Error(MFR_E_RUNTIME, "sgemm: no workspace for operand staging");
            }
            // AUTO without the memory: read in place (4-byte loads; the 256x256 tile copies them
            // straight into LDS).
            plan.stage_a = plan.stage_b = false;
            fa = fb = 0;
            if (d.tile == MFR_TILE_AUTO) {
                single_region(plan, choose(p.m, p.n, p.k, p.batch_count, s.compute_units,
                                           MFR_TILE_AUTO, 1, plan.c0, plan.ak, plan.bk,
                                           thin_b_layout(p, plan, p.m, p.n), big_tile_ok(plan)));
            }
        }
    }
    float* partial = partial_floats(plan) > 0 ? ws : nullptr;
    if (plan.stage_b) {
        stage_operand(ob, ws + partial_floats(plan) + fa, p, s.stream);
        p.b = ob.base;
        vb = 4;
    }
    // A staged K-major A (rows of k floats) beside a peeled strip of at most 8 columns over all of
    // its rows (the MLP's 4093 x 3): the strip's launch reads A's rows once and writes the copy
    // too, instead of a copy launch and then the strip reading the copy.
    int fused = -1;
    if (plan.stage_a && plan.ak && va == 1 && p.batch_count == 1) {
        for (int i = 1; i < plan.region_count; ++i) {
            const Region& r = plan.regions[i];
            bool along_n = false;
            if (r.tile == MFR_TILE_THIN && r.m_off == 0 && r.m == p.m &&
                thin_possible(r.m, r.n, plan.ak, plan.bk, &along_n) && along_n &&
                p.k * (r.n <= 1 ? 1 : r.n <= 2 ? 2 : r.n <= 4 ? 4 : kThinCols) <=
                    kStripLdsFloats) {
                fused = i;
                break;
            }
        }
    }
    if (fused >= 0) {
        float* dst = ws + partial_floats(plan);
        launch_region(plan, p, plan.regions[fused], va, vb, partial, s.compute_units, s.stream,
                      dst, round4(oa.inner));
        repoint_staged(oa, dst, p);
        p.a = oa.base;
        va = 4;
    } else if (plan.stage_a) {
        stage_operand(oa, ws + partial_floats(plan), p, s.stream);
        p.a = oa.base;
        va = 4;
    }
    for (int i = 0; i < plan.region_count; ++i) {
        if (i != fused) {
            launch_region(plan, p, plan.regions[i], va, vb, partial, s.compute_units, s.stream);
        }
    }
}

} // namespace

// ---- the no-allocation entry point ------------------------------------------------------------
//
// mfr_sgemm_noalloc's workspace: one fixed array per device, held until the process ends. Host
// code never uses its name as an address (in host code it names a host-side stand-in): each
// device's address comes from hipGetSymbolAddress, taken once per device with that device
// current, and only that address reaches kernels.
static constexpr size_t kScratchBytes = MFR_SGEMM_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxScratchDevices = 64;
static std::mutex scratch_mutex;
static float* scratch_address[kMaxScratchDevices] = {};

// The device address of `scratch` on s's device (current, as stream_of made it).
static float* scratch_on(const mfr_stream& s) {
    mfr::require(s.device >= 0 && s.device < kMaxScratchDevices,
                 "sgemm_noalloc: device index out of range");
    std::lock_guard<std::mutex> hold(scratch_mutex);
    if (scratch_address[s.device] == nullptr) {
        void* address = nullptr;
        mfr::check(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)),
                   "hipGetSymbolAddress(scratch)");
        scratch_address[s.device] = static_cast<float*>(address);
    }
    return scratch_address[s.device];
}

extern "C" {

int mfr_sgemm_noalloc(mfr_stream_t stream, const mfr_gemm_desc* desc) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(desc != nullptr, "sgemm_noalloc: null descriptor");
        run_sgemm(s, *desc, scratch_on(s), kScratchBytes);
    });
}

int mfr_sgemm(mfr_stream_t stream, const mfr_gemm_desc* desc) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(desc != nullptr, "sgemm: null descriptor");
        run_sgemm(s, *desc);
    });
}

int mfr_sgemm_plan(int device, const mfr_gemm_desc* desc, int32_t* tile, int32_t* stage,
                   int32_t* splits, int32_t* regions) {
    return mfr::guarded([&] {
        mfr::require(desc != nullptr && tile != nullptr && stage != nullptr && splits != nullptr &&
                         regions != nullptr,
                     "sgemm_plan: null argument");
        int cus = 0;
        const int status = mfr_get_device_info(device, nullptr, 0, nullptr, &cus, nullptr);
        if (status != MFR_OK) {
            throw mfr::Error(status, mfr_last_error());
        }
        const Plan plan = plan_sgemm(*desc, cus);
        *tile = plan.empty ? MFR_TILE_AUTO : plan.regions[0].tile;
        *stage = plan.stage_a || plan.stage_b ? MFR_STAGE_ALWAYS : MFR_STAGE_NEVER;
        *splits = plan.empty ? 0 : plan.regions[0].splits;
        *regions = plan.empty ? 0 : plan.region_count;
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
