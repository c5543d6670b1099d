// Device code of the thin GEMM path: products with at most 8 output columns (or, transposed, 8
// output rows), which the MFMA tiles would pad to 64 and more. Included by gemm.hip, which picks
// the path and sets up the parameters.
//
// The product is C'[rows, cols] = A'[rows, k] B'[k, cols] with cols <= 8, in general strides, so
// one kernel serves both orientations: C = A B with n <= 8 (A' = A, B' = B), and C^T = B^T A^T
// with m <= 8 (A' = B^T, B' = A^T, C' = C^T). The work is streaming A' from HBM once (as the gemv
// kernels stream their matrix); B' (at most 8 columns) is read through the caches by every row,
// one value at a time or, where its rows allow, as 8- or 16-byte pieces of a row (VB below).
// A' rows must run along k (unit stride along k): each wavefront takes kThinRowsPerWave rows, its
// lanes stride through k (16-byte loads when the rows allow), and the wavefront sums its lanes at
// the end.
// Each output is act(fl(fl(fl(alpha * sum) + fl(beta * C0)) + bias)), the MFMA epilogue's
// roundings; the sum is fp32 in an order of its own (exact, in any order, on quarter integers).
#pragma once

#include "common.hpp"

namespace mfr::gemm {

constexpr int kThinCols = 8;        // most output columns (rows, transposed) the path takes
constexpr int kThinRowsPerWave = 4;
constexpr int kThinWaves = 2;
constexpr int kThinThreads = 64 * kThinWaves;
constexpr int kThinDotRows = kThinRowsPerWave * kThinWaves; // rows per workgroup
constexpr int kThinUnroll = 2;

// Steps of 64 * VA depths a wavefront loads before it adds any. 4-byte loads take 4 times the
// steps for the same depths, so as many loads are in flight per round trip to memory. The count
// is part of the arithmetic: each lane adds its depths in increasing order, and the steps past k
// add 0 * 0, which turns a sum of -0 into +0, so strip_stage_kernel takes the same count.
constexpr int thin_unroll(int va, int c) {
    return va == 4 ? kThinUnroll : c == kThinCols ? 2 * kThinUnroll : 4 * kThinUnroll;
}

struct ThinParams {
    const float* a;
    const float* b;
    float* c;
    const float* c0;   // null when beta * C0 is not added
    const float* bias; // may be null
    int64_t rows, cols, k;
    int64_t a_rs, a_cs; // A'(r, p) at a + r*a_rs + p*a_cs
    int64_t b_rs, b_cs; // B'(p, j) at b + p*b_rs + j*b_cs
    int64_t c_rs, c_cs, c0_rs, c0_cs;
    int64_t bias_rs, bias_cs; // bias'(r, j) at bias + r*bias_rs + j*bias_cs
    int64_t batch[MFR_MAX_BATCH_DIMS];
    int64_t a_bs[MFR_MAX_BATCH_DIMS], b_bs[MFR_MAX_BATCH_DIMS];
    int64_t c_bs[MFR_MAX_BATCH_DIMS], c0_bs[MFR_MAX_BATCH_DIMS];
    int32_t batch_dims;
    int32_t act;
    int64_t blocks_per_batch;
    float alpha, beta;
    // strip_stage_kernel only: A' row r is also copied to stage + r * stage_rs, zero-padded from
    // k to stage_rs (one matrix, no batch).
    float* stage;
    int64_t stage_rs;
};

// Offsets of batch matrix `index` (linear order) into A', B', C' and C0'.
struct ThinBatch {
    const float* a;
    const float* b;
    float* c;
    const float* c0;
};

__device__ inline ThinBatch thin_batch(const ThinParams& p, int64_t index) {
    int64_t off_a = 0, off_b = 0, off_c = 0, off_c0 = 0;
    for (int d = p.batch_dims - 1; d >= 0; --d) {
        const int64_t i = index % p.batch[d];
        index /= p.batch[d];
        off_a += i * p.a_bs[d];
        off_b += i * p.b_bs[d];
        off_c += i * p.c_bs[d];
        off_c0 += i * p.c0_bs[d];
    }
    return ThinBatch{p.a + off_a, p.b + off_b, p.c + off_c,
                     p.c0 != nullptr ? p.c0 + off_c0 : nullptr};
}

__device__ inline void thin_store(const ThinParams& p, const ThinBatch& t, int64_t r, int64_t j,
                                  float sum) {
    float v = p.alpha * sum;
    if (t.c0 != nullptr) {
        const float scaled = p.beta * t.c0[r * p.c0_rs + j * p.c0_cs];
        v = v + scaled;
    }
    if (p.bias != nullptr) {
        v = v + p.bias[r * p.bias_rs + j * p.bias_cs];
    }
    t.c[r * p.c_rs + j * p.c_cs] = mfr::dev::activate(v, p.act);
}

// VA = 4: 16-byte loads of A' (a_rs and the batch strides multiples of 4, a 16-byte aligned, and
// either k % 4 == 0 or A' staged with its lines zero-padded to a multiple of 4).
// C: the column count rounded up to 1, 2, 4 or 8; columns from p.cols to C are neither loaded
// nor stored. B' values come from the caches (shared by every row).
// VB: B' rows are read as 8-byte (C = 2) or 16-byte (C = 4, 8) pieces of C columns. The launch
// takes this form only where B' has unit column stride, its rows and batches start aligned to
// the piece, and the C columns exist in memory (exactly C columns, or a staged copy whose lines
// are zero-padded to a multiple of 4). Each lane reads rows of its own depths, so per-element
// loads make C cache-line accesses per row: those, not the bytes, set the time (16384 x 4 x 4096:
// 124.7 against 50.9 us).
template <int VA, int C, bool VB = false>
__global__ __launch_bounds__(kThinThreads) void thin_dot_kernel(ThinParams p) {
    static_assert(C == 1 || C == 2 || C == 4 || C == kThinCols, "C is 1, 2, 4 or 8");
    static_assert(!VB || C % 2 == 0, "B' pieces need 2, 4 or 8 columns");
    const int64_t batch_index = blockIdx.x / p.blocks_per_batch;
    const ThinBatch t = thin_batch(p, batch_index);
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int64_t row0 =
        (blockIdx.x % p.blocks_per_batch) * kThinDotRows + wave * kThinRowsPerWave;
    const int cols = static_cast<int>(p.cols);
    float acc[kThinRowsPerWave][C] = {};
    const float* a_row[kThinRowsPerWave];
    bool valid[kThinRowsPerWave];
#pragma unroll
    for (int r = 0; r < kThinRowsPerWave; ++r) {
        valid[r] = row0 + r < p.rows;
        a_row[r] = t.a + (valid[r] ? row0 + r : 0) * p.a_rs;
    }
    // kUnroll steps of 64 * VA depths: every load of a group is issued before any is used;
    // steps past k load zeros and add 0 * 0.
    constexpr int kUnroll = thin_unroll(VA, C);
    constexpr int kStep = 64 * VA * kUnroll; // depths per group
    for (int64_t base = static_cast<int64_t>(lane) * VA; base < p.k; base += kStep) {
        float a[kUnroll][kThinRowsPerWave][VA];
        float b[kUnroll][VA][C];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t kk = base + u * 64 * VA;
            const bool in_k = kk < p.k;
#pragma unroll
            for (int r = 0; r < kThinRowsPerWave; ++r) {
                const bool ok = valid[r] && in_k;
                if constexpr (VA == 4) {
                    const float4 v =
                        ok ? mfr::dev::load_streaming(a_row[r] + kk) : make_float4(0.f, 0.f, 0.f, 0.f);
                    a[u][r][0] = v.x;
                    a[u][r][1] = v.y;
                    a[u][r][2] = v.z;
                    a[u][r][3] = v.w;
                } else {
                    a[u][r][0] = ok ? a_row[r][kk] : 0.0f;
                }
            }
#pragma unroll
            for (int v = 0; v < VA; ++v) {
                // A staged operand's lines are padded to a multiple of 4 (the A' values past k
                // read its zeros), but B' has no depth kk + v >= k: those are not read.
                const bool depth = kk + v < p.k;
                if constexpr (VB && C == 2) {
                    const float2 w =
                        depth ? *reinterpret_cast<const float2*>(t.b + (kk + v) * p.b_rs)
                              : make_float2(0.f, 0.f);
                    b[u][v][0] = w.x;
                    b[u][v][1] = 1 < cols ? w.y : 0.0f;
                } else if constexpr (VB) {
#pragma unroll
                    for (int h = 0; h < C / 4; ++h) {
                        const float4 w =
                            depth ? *reinterpret_cast<const float4*>(t.b + (kk + v) * p.b_rs + 4 * h)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
                        b[u][v][4 * h + 0] = 4 * h + 0 < cols ? w.x : 0.0f;
                        b[u][v][4 * h + 1] = 4 * h + 1 < cols ? w.y : 0.0f;
                        b[u][v][4 * h + 2] = 4 * h + 2 < cols ? w.z : 0.0f;
                        b[u][v][4 * h + 3] = 4 * h + 3 < cols ? w.w : 0.0f;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < C; ++j) {
                        b[u][v][j] = depth && j < cols ? t.b[(kk + v) * p.b_rs + j * p.b_cs] : 0.0f;
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
            for (int v = 0; v < VA; ++v) {
#pragma unroll
                for (int r = 0; r < kThinRowsPerWave; ++r) {
#pragma unroll
                    for (int j = 0; j < C; ++j) {
                        acc[r][j] = __builtin_fmaf(a[u][r][v], b[u][v][j], acc[r][j]);
                    }
                }
            }
        }
    }
    // Wavefront sums: every lane ends with every total; lane r*C + j stores output (r, j).
    // (A halving exchange, each lane keeping half of its values per step, ran slower: 10.2
    // against 7.9 us on 4093 x 3 x 1023.)
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < kThinRowsPerWave; ++r) {
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const float v = mfr::dev::butterfly_sum(acc[r][j]);
            mine = lane == r * C + j ? v : mine;
        }
    }
    const int r = lane / C;
    const int j = lane % C;
    if (r < kThinRowsPerWave && row0 + r < p.rows && j < cols) {
        thin_store(p, t, row0 + r, j, mine);
    }
}

// thin_dot_kernel<4, kThinCols, true>'s products and sums (every lane adds its depths in the same
// order, so the same bits) with B' staged through LDS. There each wavefront reads all of B' (k
// rows of 32 bytes) through the caches, twice the bytes of its own 4 rows of A, and with 8
// columns those reads, not A's stream, set the time. Here a workgroup of WAVES wavefronts copies
// each group of kStep depths of B' into LDS once (double-buffered, one barrier per group), and
// every lane reads its 4 depths' rows from there. The launch takes it for 8 columns in 16-byte
// pieces from kThinLdsMinRows rows. On one MI355X, against thin_dot_kernel (with 2 and 8
// wavefronts in brackets): 16384 x 8 x 4096 91 -> 55.6 us (60.6, 63.1); 65536 x 8 x 512
// 44 -> 31.6 us (46.9, 33.4); 16384 x 8 x 1000 25.7 -> 15.3 us; 4096 x 8 x 1024 10.9 -> 8.4 us;
// 1024 x 8 x 8192 34.7 -> 34.0 us (30.5, 42.0); 3 x 8 x 5 5.3 -> 6.3 us.
constexpr int kThinLdsWaves = 4;
constexpr int64_t kThinLdsMinRows = 16;
template <int WAVES> constexpr int thin_lds_rows() { return kThinRowsPerWave * WAVES; }

template <int WAVES>
__global__ __launch_bounds__(64 * WAVES) void thin_dot_lds_kernel(ThinParams p) {
    constexpr int VA = 4;
    constexpr int C = kThinCols;
    constexpr int THREADS = 64 * WAVES;
    constexpr int kUnroll = thin_unroll(VA, C);
    constexpr int kStep = 64 * VA * kUnroll; // depths per group
    static_assert(kStep % THREADS == 0, "whole B' rows per thread per group");
    constexpr int kFills = kStep / THREADS;  // B' rows each thread copies per group
    // A group's LDS image: its depths in fours (one lane's), 4 C floats each, padded by 4 floats
    // so that the 16 lanes of one 16-byte read pass hit 16 different 4-bank quads.
    constexpr int kQuadPitch = 4 * C + 4;
    constexpr int kGroupFloats = kStep / 4 * kQuadPitch;
    __shared__ __align__(16) float b_lds[2][kGroupFloats];

    const int64_t batch_index = blockIdx.x / p.blocks_per_batch;
    const ThinBatch t = thin_batch(p, batch_index);
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int64_t row0 = (blockIdx.x % p.blocks_per_batch) * thin_lds_rows<WAVES>() +
                         wave * kThinRowsPerWave;
    const int cols = static_cast<int>(p.cols);
    float acc[kThinRowsPerWave][C] = {};
    const float* a_row[kThinRowsPerWave];
    bool valid[kThinRowsPerWave];
#pragma unroll
    for (int r = 0; r < kThinRowsPerWave; ++r) {
        valid[r] = row0 + r < p.rows;
        a_row[r] = t.a + (valid[r] ? row0 + r : 0) * p.a_rs;
    }
    // B' row `group + i * THREADS + threadIdx.x` of a group (zeros past k) into registers, then
    // into the group's LDS image.
    float4 w[kFills][2];
    const auto fetch = [&](int64_t group) {
#pragma unroll
        for (int i = 0; i < kFills; ++i) {
            const int64_t d = group + i * THREADS + threadIdx.x;
            if (d < p.k) {
                const float* src = t.b + d * p.b_rs;
                w[i][0] = *reinterpret_cast<const float4*>(src);
                w[i][1] = *reinterpret_cast<const float4*>(src + 4);
            } else {
                w[i][0] = make_float4(0.f, 0.f, 0.f, 0.f);
                w[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    const auto put = [&](int buffer) {
#pragma unroll
        for (int i = 0; i < kFills; ++i) {
            const int row = i * THREADS + static_cast<int>(threadIdx.x);
            float* dst = b_lds[buffer] + (row / 4) * kQuadPitch + (row % 4) * C;
            *reinterpret_cast<float4*>(dst) = w[i][0];
            *reinterpret_cast<float4*>(dst + 4) = w[i][1];
        }
    };
    fetch(0);
    put(0);
    __syncthreads();
    int buffer = 0;
    for (int64_t group = 0; group < p.k; group += kStep) {
        const bool more = group + kStep < p.k;
        if (more) {
            fetch(group + kStep);
        }
        // This lane's depths as thin_dot_kernel takes them: base, base + 64 VA, ... A lane whose
        // first depth is past k takes no step there (it would add 0 * 0, turning -0 into +0).
        const int64_t base = group + static_cast<int64_t>(lane) * VA;
        if (base < p.k) {
            float a[kUnroll][kThinRowsPerWave][VA];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t kk = base + u * 64 * VA;
                const bool in_k = kk < p.k;
#pragma unroll
                for (int r = 0; r < kThinRowsPerWave; ++r) {
                    const float4 v = valid[r] && in_k ? mfr::dev::load_streaming(a_row[r] + kk)
                                                      : make_float4(0.f, 0.f, 0.f, 0.f);
                    a[u][r][0] = v.x;
                    a[u][r][1] = v.y;
                    a[u][r][2] = v.z;
                    a[u][r][3] = v.w;
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const float* quad = b_lds[buffer] + (u * 64 + lane) * kQuadPitch;
#pragma unroll
                for (int v = 0; v < VA; ++v) {
                    float b[C];
#pragma unroll
                    for (int h = 0; h < C / 4; ++h) {
                        const float4 x = *reinterpret_cast<const float4*>(quad + v * C + 4 * h);
                        b[4 * h + 0] = 4 * h + 0 < cols ? x.x : 0.0f;
                        b[4 * h + 1] = 4 * h + 1 < cols ? x.y : 0.0f;
                        b[4 * h + 2] = 4 * h + 2 < cols ? x.z : 0.0f;
                        b[4 * h + 3] = 4 * h + 3 < cols ? x.w : 0.0f;
                    }
#pragma unroll
                    for (int r = 0; r < kThinRowsPerWave; ++r) {
#pragma unroll
                        for (int j = 0; j < C; ++j) {
                            acc[r][j] = __builtin_fmaf(a[u][r][v], b[j], acc[r][j]);
                        }
                    }
                }
            }
        }
        if (more) {
            put(buffer ^ 1);
        }
        __syncthreads();
        buffer ^= 1;
    }
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < kThinRowsPerWave; ++r) {
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const float v = mfr::dev::butterfly_sum(acc[r][j]);
            mine = lane == r * C + j ? v : mine;
        }
    }
    const int r = lane / C;
    const int j = lane % C;
    if (r < kThinRowsPerWave && row0 + r < p.rows && j < cols) {
        thin_store(p, t, row0 + r, j, mine);
    }
}

// A peeled strip of at most 8 columns over every row of a K-major A whose rows 16-byte loads
// cannot take, and the staging of that A for the MFMA tiles, in one launch: each wavefront takes
// one row of A' = A, copies it to p.stage (zero-padded from k to stage_rs) as it reads it, and sums
// its products with B', which the workgroup keeps in LDS (k x C floats, filled once). The sums are
// thin_dot_kernel<1, C>'s bit for bit: lane l adds depths l, l + 64, ... in increasing order in
// groups of thin_unroll(1, C) steps, then the wavefront's butterfly. One matrix, no batch.
constexpr int kStripWaves = 16;
constexpr int64_t kStripLdsFloats = 16384; // k * C at most (64 KiB of LDS)

template <int C>
__global__ __launch_bounds__(64 * kStripWaves) void strip_stage_kernel(ThinParams p) {
    static_assert(C == 1 || C == 2 || C == 4 || C == kThinCols, "C is 1, 2, 4 or 8");
    extern __shared__ float b_lds[]; // B'(d, j) at b_lds[d * C + j], zero past p.cols
    constexpr int kUnroll = thin_unroll(1, C);
    constexpr int64_t kStep = 64 * kUnroll;
    const int lane = threadIdx.x % 64;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kStripWaves + threadIdx.x / 64;
    const bool active = row < p.rows;
    const float* a_row = p.a + (active ? row : 0) * p.a_rs;
    // A group of depths of this lane's row (zeros past k); the next group is always in flight
    // while the current one is copied and added, and the first while B' fills LDS.
    const auto load_group = [&](int64_t base, float (&a)[kUnroll]) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t kk = base + 64 * u;
            a[u] = active && kk < p.k ? a_row[kk] : 0.0f;
        }
    };
    float a[kUnroll];
    load_group(lane, a);
    const int cols = static_cast<int>(p.cols);
    // B' into LDS: a thread issues its loads for kFill entries before storing any, so the fill
    // waits for one round trip to memory per kFill entries instead of one per entry (the MLP's
    // strip, 4093 x 3 x 1023: 11.5-11.9 -> 10.5-11.0 us).
    constexpr int kFill = 8;
    const int64_t entries = p.k * C;
    for (int64_t i0 = threadIdx.x; i0 < entries; i0 += kFill * blockDim.x) {
        float v[kFill];
#pragma unroll
        for (int u = 0; u < kFill; ++u) {
            const int64_t i = i0 + static_cast<int64_t>(u) * blockDim.x;
            const int64_t d = i / C;
            const int j = static_cast<int>(i % C);
            v[u] = i < entries && j < cols ? p.b[d * p.b_rs + j * p.b_cs] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kFill; ++u) {
            const int64_t i = i0 + static_cast<int64_t>(u) * blockDim.x;
            if (i < entries) {
                b_lds[i] = v[u];
            }
        }
    }
    __syncthreads();
    if (!active) {
        return;
    }
    float* copy = p.stage + row * p.stage_rs;
    float acc[C] = {};
    for (int64_t base = lane; base < p.k; base += kStep) {
        float next[kUnroll];
        load_group(base + kStep, next);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t kk = base + 64 * u;
            if (kk < p.k) {
                copy[kk] = a[u];
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t kk = base + 64 * u;
            float b[C];
            if (kk < p.k) {
                if constexpr (C >= 4) {
#pragma unroll
                    for (int h = 0; h < C / 4; ++h) {
                        const float4 w = *reinterpret_cast<const float4*>(b_lds + kk * C + 4 * h);
                        b[4 * h + 0] = w.x;
                        b[4 * h + 1] = w.y;
                        b[4 * h + 2] = w.z;
                        b[4 * h + 3] = w.w;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < C; ++j) {
                        b[j] = b_lds[kk * C + j];
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < C; ++j) {
                    b[j] = 0.0f;
                }
            }
#pragma unroll
            for (int j = 0; j < C; ++j) {
                acc[j] = __builtin_fmaf(a[u], b[j], acc[j]);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            a[u] = next[u];
        }
    }
    if (p.k + lane < p.stage_rs) {
        copy[p.k + lane] = 0.0f; // the padding (fewer than 4 floats)
    }
    float mine = 0.0f;
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const float v = mfr::dev::butterfly_sum(acc[j]);
        mine = lane == j ? v : mine;
    }
    if (lane < cols) {
        const ThinBatch t{p.a, p.b, p.c, p.c0};
        thin_store(p, t, row, lane, mine);
    }
}

} // namespace mfr::gemm
