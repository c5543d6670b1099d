// Device code of the panel path (MFR_TILE_PANEL): products with a short depth (k <= 64) and a
// large output, such as attention's scores q k^T (128 x [1024 x 64] x [64 x 1024], 512 MiB of
// output for 17 GFLOP). gemm.hip picks the path (panel_fits) and sets up the parameters;
// panel.hip launches it.
//
// On the tile kernels every workgroup loads its operands, multiplies, stores its tile and exits,
// and __syncthreads() before each depth slice waits for every store the workgroup has issued
// (gfx9 counts vector loads and stores on one counter, vmcnt, and the barrier's release fence
// waits for it to reach 0). A CU's workgroups then compute together and store together: the
// product took its MFMA time plus its store time. Here a workgroup keeps its operand rows and
// streams the other operand and the output past them:
//   - A workgroup of 8 wavefronts owns a panel of 256 rows of A (32 per wavefront, held in
//     registers as the MFMA fragments for the whole kernel) and walks the columns of C in tiles of
//     64: the matching 64 rows of B (K-major) come into LDS by direct-to-LDS buffer loads, double
//     buffered, and each wavefront multiplies its 32 x 64 block (two 32x32 accumulators of
//     v_mfma_f32_32x32x2_f32, the tile kernels' depth permutation, so the same sums in the same
//     order as every tile: bit-identical results) and stores it with non-temporal buffer stores.
//   - The loop never waits for its stores: before each tile's barrier a wavefront waits only until
//     its copy of the next B tile has landed (vmcnt counts in issue order, so that is "all but the
//     last tile's stores", the immediate kStoresPerTile) and the barrier is a bare s_barrier.
//     Stores drain while the next tile's MFMAs run.
//   - Workgroups start their column walk at different tiles ((4 panel + batch) mod tiles), so the
//     stores in flight at any moment spread over the output instead of all hitting the same
//     columns (config 5's scores, store-only: 136 -> 110 us).
//   - Rows past m are dropped by the store resource's record count (it ends at row m); columns
//     past n get an offset past it; depths past k and B rows past n load as zeros.
//   - Under the causal flag (MFR_GEMM_CAUSAL, attention's scores) every output with column > row
//     is -inf, and a wavefront's 32 x 64 block that lies wholly above the diagonal skips its
//     MFMAs (about half of config 5's scores). A workgroup then takes 128 rows from the top and
//     their mirror image from the bottom instead of one 256-row panel, so that every SIMD has the
//     same products to compute.
//   - The scores' form (alpha and the mask only) fits 126 VGPRs: 4 wavefronts per SIMD, two
//     workgroups per CU; with beta * C0 or a bias (FULL) 2.
// Measured on config 5's scores (one MI355X): 151-161 us against 204-216 us for the 128x64 tile,
// bit for bit the same (165-173 us with 2 wavefronts per SIMD); 116 us under the causal mask
// (148 us with each workgroup on one contiguous panel: the CUs holding the bottom panels computed
// nearly every block).
// The rest is the power limit: under MFMA work and the 512 MiB store stream together the clock
// drops to ~1.94 GHz (2.21 GHz with the stores taken out, where the same loop runs in 124-129
// us), and at 1.94 GHz the MFMA work alone takes 135 us.
#pragma once

#include "gemm_kernel.hpp"

namespace mfr::gemm {

constexpr int kPanelWaves = 8;
constexpr int kPanelRows = 32 * kPanelWaves; // rows of A per workgroup
constexpr int kPanelCols = 64;               // columns of C per tile
constexpr int kPanelMaxDepth = 64;
constexpr int kPanelThreads = 64 * kPanelWaves;
constexpr uint32_t kPanelLimit = 0x80000000u; // an offset past every record count

// Runs C = alpha op(A) op(B) (+ beta C0) (+ bias) for q on the panel path (panel.hip).
void launch_panel(const GemmParams& q, bool nt, int cus, hipStream_t stream);

struct PanelParams {
    GemmParams g;
    int32_t panels;    // row panels of kPanelRows per matrix
    int32_t nblocks;   // column tiles of kPanelCols per matrix
    int32_t chunks;    // column ranges per panel (each a workgroup of its own)
    int32_t per_chunk; // tiles per range
};

// s_waitcnt with vmcnt N and the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8). The count is of the vector memory operations issued before
// it, so none of them may be moved past it: the empty asm statement keeps the compiler from
// sinking the tile's stores below the wait (which would let the wait pass before the LDS copy it
// is there for had landed).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// A workgroup barrier without the release fence of __syncthreads() (which waits for vmcnt 0,
// the stores included). The empty asm statements keep the compiler from moving memory accesses
// across it; the LDS tiles' copies are waited for explicitly before it.
__device__ __forceinline__ void bare_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// KG: 8-deep depth groups held (k <= 8 KG). NT: non-temporal stores (outputs larger than the
// last-level cache whose rows start on 128-byte lines). FULL: the epilogue with beta * C0 and a
// bias; without it (the scores' case) only alpha and the causal mask, in the store loop itself,
// which keeps the kernel at 4 wavefronts per SIMD.
template <int KG, bool NT, bool FULL>
__global__ __launch_bounds__(kPanelThreads, FULL ? 2 : 4) void sgemm_panel_kernel(PanelParams pp) {
    const GemmParams& p = pp.g;
    constexpr int KT = 8 * KG;
    constexpr int PITCH = KT + 4;               // LDS row pitch: the tile kernels' K-major image
    constexpr int kTileFloats = kPanelCols * PITCH;
    constexpr int kInstr = kTileFloats / 256;   // 1 KiB wave-instructions per tile copy
    constexpr int kPerWave = (kInstr + kPanelWaves - 1) / kPanelWaves;
    static_assert(kTileFloats % 256 == 0, "a tile image is whole wave-instructions");
    constexpr int kStoresPerTile = 32;          // buffer stores per wavefront per tile
    // One LDS object per buffer, so the compiler sees that the copy into one does not write the
    // one the MFMAs read.
    __shared__ __align__(16) float tile0[kTileFloats];
    __shared__ __align__(16) float tile1[kTileFloats];

    // Workgroup -> (batch, column range, panel), consecutive logical indices on one XCD (the
    // hardware sends workgroup i to XCD i % 8), panels fastest: the panels of a batch share its
    // B tiles in that XCD's L2.
    const uint32_t total = gridDim.x;
    const uint32_t hw = blockIdx.x;
    const uint32_t per_xcd = total / 8;
    const uint32_t logical = hw < per_xcd * 8 ? (hw % 8) * per_xcd + hw / 8 : hw;
    const uint32_t panel = logical % static_cast<uint32_t>(pp.panels);
    const uint32_t rest = logical / static_cast<uint32_t>(pp.panels);
    const uint32_t chunk = rest % static_cast<uint32_t>(pp.chunks);
    uint32_t batch_index = rest / static_cast<uint32_t>(pp.chunks);
    const uint32_t batch_linear = batch_index;
    int64_t off_a = 0, off_b = 0, off_c = 0, off_c0 = 0;
    for (int d = p.batch_dims - 1; d >= 0; --d) {
        const uint32_t extent = static_cast<uint32_t>(p.batch[d]);
        const int64_t idx = batch_index % extent;
        batch_index /= extent;
        off_a += idx * p.a_bs[d];
        off_b += idx * p.b_bs[d];
        off_c += idx * p.c_bs[d];
        off_c0 += idx * p.c0_bs[d];
    }

    const int lane = static_cast<int>(__lane_id());
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / 64));
    const int half = lane / 32;
    const int r32 = lane % 32;
    // This wavefront's 32-row block. Without the causal mask, block 8 panel + wave. Under it the
    // blocks near the top skip most of their column tiles and those near the bottom almost none,
    // so panel p takes blocks 4p .. 4p + 3 from the top (wavefronts 0-3) and their mirror images
    // from the bottom of the 8 panels blocks (wavefronts 4-7): wavefronts w and w + 4 share a
    // SIMD, and every SIMD then has the same products to compute (17 of the 32 tile-blocks of its
    // two wavefronts when the matrix is square). Blocks past m compute nothing that is stored.
    const bool causal = p.causal != 0;
    const int block = !causal    ? 8 * static_cast<int>(panel) + wave
                      : wave < 4 ? 4 * static_cast<int>(panel) + wave
                                 : 8 * pp.panels - 1 - (4 * static_cast<int>(panel) + wave - 4);
    const int64_t row0 = static_cast<int64_t>(block) * 32;

    const int t_first = static_cast<int>(chunk) * pp.per_chunk;
    const int t_left = pp.nblocks - t_first;
    const int t_count = t_left < pp.per_chunk ? t_left : pp.per_chunk;
    if (t_count <= 0) {
        return; // uniform over the workgroup: no barrier is left waiting
    }
    const int rot =
        static_cast<int>((4 * panel + batch_linear) % static_cast<uint32_t>(t_count));
    const auto col_tile = [&](int i) { // the i-th tile this workgroup walks
        const int j = i + rot;
        return t_first + (j >= t_count ? j - t_count : j);
    };

    // B tile copies: image float f = (instruction * 64 + lane) * 4 is row f / PITCH (a column of
    // C) and depth f % PITCH; pads and depths past k get the limit and load zeros, rows past n
    // fall outside the tile's record count.
    const float* b_mat = p.b + off_b;
    uint32_t b_off[kPerWave];
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        const int f = ((wave * kPerWave + j) * 64 + lane) * 4;
        const int row = f / PITCH;
        const int at = f - row * PITCH;
        b_off[j] = at < p.k ? static_cast<uint32_t>((row * p.b_cs + at) * 4) : kPanelLimit;
    }
    const auto issue = [&](float* dst, int i) {
        const int64_t n0 = static_cast<int64_t>(col_tile(i)) * kPanelCols;
        const int64_t rows = p.n - n0 < kPanelCols ? p.n - n0 : kPanelCols;
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(b_mat + n0 * p.b_cs), 0, static_cast<int>(rows * p.b_cs * 4),
            kBufferWord3);
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int instr = wave * kPerWave + j;
            if (kInstr % kPanelWaves != 0 && instr >= kInstr) {
                break; // uniform: this wave's share ended
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst + instr * 256, 16,
                                                     static_cast<int>(b_off[j]), 0, 0, 0);
        }
    };
    issue(tile0, 0);

    // A fragments for the whole walk: row row0 + r32, depths 8g + 4 half .. + 3 (the depth
    // permutation of the tile kernels' K-major fragments).
    float4 af[KG];
    {
        const int64_t row = row0 + r32;
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(p.a + off_a), 0, 0x7fffffff, kBufferWord3);
        const uint32_t row_off =
            row < p.m ? static_cast<uint32_t>(row * p.a_rs * 4) : kPanelLimit;
#pragma unroll
        for (int g = 0; g < KG; ++g) {
            const int d = 8 * g + 4 * half;
            const uint32_t off = d < p.k ? row_off + static_cast<uint32_t>(d * 4) : kPanelLimit;
            const auto raw = __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(off),
                                                                   0, 0);
            af[g] = make_float4(__uint_as_float(raw[0]), __uint_as_float(raw[1]),
                                __uint_as_float(raw[2]), __uint_as_float(raw[3]));
        }
    }

    // Element e of accumulator j is row row0 + 4 half + dr(e), dr(e) = 8(e/4) + e%4, column
    // n0 + 32 j + r32.
    float* const c_mat = p.c + off_c;
    const float* const c0_mat = p.c0 != nullptr && p.beta != 0.0f ? p.c0 + off_c0 : nullptr;
    const uint32_t lane_c = static_cast<uint32_t>((4 * half * p.c_rs + r32) * 4);
    const uint32_t lane_c0 = static_cast<uint32_t>((4 * half * p.c0_rs + r32) * 4);
    const uint32_t c_rs4 = static_cast<uint32_t>(p.c_rs * 4);
    const uint32_t c0_rs4 = static_cast<uint32_t>(p.c0_rs * 4);
    const float alpha = p.alpha;
    const float beta = p.beta;
    const float* const bias = p.bias;

    const auto compute_store = [&](const float* tile, int i) {
        const int64_t n0 = static_cast<int64_t>(col_tile(i)) * kPanelCols;
        floatx16 acc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                acc[j][e] = 0.0f;
            }
        }
        // Under the causal mask a block whose first column is past its last row is all -inf:
        // its products are not computed (uniform over the wavefront).
        const bool computed = !causal || n0 <= row0 + 31;
        const float* frag = tile + r32 * PITCH + 4 * half;
        if (computed) {
#pragma unroll
            for (int g = 0; g < KG; ++g) {
                float4 bf[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    bf[j] = *reinterpret_cast<const float4*>(frag + 32 * j * PITCH + 8 * g);
                }
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const float av =
                        s == 0 ? af[g].x : s == 1 ? af[g].y : s == 2 ? af[g].z : af[g].w;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float bv =
                            s == 0 ? bf[j].x : s == 1 ? bf[j].y : s == 2 ? bf[j].z : bf[j].w;
                        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[j], 0, 0, 0);
                    }
                }
            }
        }
        // One resource per tile at (row0, n0) whose record count ends at row m (rows past m are
        // dropped); columns past n get kPanelLimit, which stays past the record count after any
        // row step (the host keeps (m + 32) * c_rs * 4 below 2^31).
        const int64_t records = (p.m - row0) * p.c_rs - n0;
        const __amdgpu_buffer_rsrc_t c_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            c_mat + row0 * p.c_rs + n0, 0, static_cast<int>(records > 0 ? records * 4 : 0),
            kBufferWord3);
        // Each lane's offset of row row0 + 4 half and its column of block j, or past the record
        // count when that column is past n (rows then step by multiples of the row stride; the
        // per-tile value keeps the compiler from holding 32 invariant sums in registers).
        uint32_t col_c[2], col_c0[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t outside = n0 + 32 * j + r32 < p.n ? 0u : kPanelLimit;
            col_c[j] = (lane_c + 128u * j) | outside;
            col_c0[j] = (lane_c0 + 128u * j) | outside;
        }
        // -inf where column > row under the causal mask: column n0 + 32 j + r32, row row0 +
        // 4 half + dr(e), i.e. where 32 j + r32 - 4 half - dr(e) > row0 - n0 (clamped: the left
        // side lies in [-35, 63]). The value's own arithmetic is kept for the rest, so the bits
        // are those of where(keep, scores, -inf).
        const int64_t gap = row0 - n0;
        const int limit = !causal ? 64 : static_cast<int>(gap < -64 ? -64 : gap > 64 ? 64 : gap);
        const auto masked = [&](int j, int e) {
            return 32 * j + r32 - 4 * half - (8 * (e / 4) + e % 4) > limit;
        };
        const auto store = [&](int j, int e, float out) {
            const uint32_t step = static_cast<uint32_t>(8 * (e / 4) + e % 4) * c_rs4;
            const uint32_t off = col_c[j] + step;
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), c_rsrc,
                                                  static_cast<int>(off), 0, NT ? 2 : 0);
        };
        if constexpr (!FULL) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float out = alpha * acc[j][e];
                    store(j, e, masked(j, e) ? -INFINITY : out);
                }
            }
        } else {
            float bias_of[2] = {-0.0f, -0.0f}; // x + -0 is x: no bias adds nothing
            if (bias != nullptr) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t col = n0 + 32 * j + r32;
                    bias_of[j] = col < p.n ? bias[col] : 0.0f;
                }
            }
            float v[2][16];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    v[j][e] = alpha * acc[j][e];
                }
            }
            if (c0_mat != nullptr) {
                // All 32 C0 values are loaded before any is used (and before any store: C0 may
                // be C).
                const int64_t records0 = (p.m - row0) * p.c0_rs - n0;
                const __amdgpu_buffer_rsrc_t c0_rsrc = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<float*>(c0_mat + row0 * p.c0_rs + n0), 0,
                    static_cast<int>(records0 > 0 ? records0 * 4 : 0), kBufferWord3);
                float c0v[2][16];
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint32_t step = static_cast<uint32_t>(8 * (e / 4) + e % 4) * c0_rs4;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const uint32_t off = col_c0[j] + step;
                        c0v[j][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                            c0_rsrc, static_cast<int>(off), 0, 0));
                    }
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const float scaled = beta * c0v[j][e];
                        v[j][e] = v[j][e] + scaled;
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float out = v[j][e] + bias_of[j];
                    store(j, e, masked(j, e) ? -INFINITY : out);
                }
            }
        }
    };

    // The first tile is read by every wavefront and copied by all of them: all copies (and this
    // wavefront's A fragments) land before the walk starts.
    wait_vmcnt<0>();
    bare_barrier();
    // The walk, unrolled by two so each half names its buffers. Before each barrier: this
    // wavefront's copy of the next tile has landed. Only the stores issued after that copy may
    // still be in flight (vmcnt counts in order, and exactly kStoresPerTile stores follow it;
    // C0 and bias loads come between, so the wait also covers them).
    for (int i = 0;; i += 2) {
        if (i + 1 < t_count) {
            issue(tile1, i + 1);
        }
        compute_store(tile0, i);
        if (i + 1 >= t_count) {
            break;
        }
        wait_vmcnt<kStoresPerTile>();
        bare_barrier();
        if (i + 2 < t_count) {
            issue(tile0, i + 2);
        }
        compute_store(tile1, i + 1);
        if (i + 2 >= t_count) {
            break;
        }
        wait_vmcnt<kStoresPerTile>();
        bare_barrier();
    }
}

} // namespace mfr::gemm
