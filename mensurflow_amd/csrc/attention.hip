// Fused scaled dot-product attention on the fp32 matrix cores (include/mfr_rocm.h,
// mfr_attention). One kernel computes softmax(scale * q k^T, masked) v without writing the
// [.., lq, lk] scores to memory; the reference composes the same op from a batched GEMM, where(),
// softmax and a second batched GEMM (src/ops/attention.cpp:48-98).
//
// Design (a workgroup of 8 wavefronts, 4 for d = 32, 32 queries each; keys in blocks of BK):
//   - Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x2_f32: the accumulator
//     of a 32-key x 32-query block puts one query in each lane column (lanes l and l+32 hold
//     query l % 32, 16 keys each). Every per-query quantity of the softmax (running maximum,
//     running sum, rescale factor) is then lane-local, with one exchange between the two lane
//     halves per key block for the maximum.
//   - The output is also computed transposed, O^T += V^T P^T. Its B operand P^T needs, in lane l
//     at step s of depth group g, the weight of query l % 32 and key 8g + 4(l / 32) + s, which is
//     exactly accumulator element 4g + s of that lane in S^T: the probabilities feed the second
//     product straight from registers, with no shuffle and no trip through LDS.
//   - q's fragments stay in registers for the whole key loop. K and V tiles are double-buffered
//     in LDS through the GEMM's slice loader: K [keys][d+4] (K-major, 16-byte fragment reads),
//     V [keys][d+8] (read as V^T fragments, four 4-byte reads).
//   - Causal attention skips, per wavefront, every key block lying wholly above its queries'
//     diagonal, and the key loop stops at the workgroup's last query. Workgroups are
//     issued longest first (the last query blocks of every batch entry) so the short ones fill
//     the tail.
//   - The result is scaled by the reciprocal of the row sum, staged through LDS and stored as
//     16-byte rows.
//   - attention16_kernel (below) is the same op with 16 queries per wavefront on the 16x16x4
//     MFMA, at 4 wavefronts per SIMD; it takes causal d = 64 on large grids.
#include "gemm_kernel.hpp"

#include <cmath>

namespace {

using mfr::gemm::floatx16;
using mfr::gemm::SliceLoader;

constexpr int kWaves = 4; // wavefronts of 32 queries per workgroup, by default

// Wavefronts per workgroup by head size: 8 for d = 64 and 128, where one K/V tile then serves
// 256 queries (8 x 16 x 1024, causal: d = 64 189-191 us against 199-205 us with 4; d = 128
// 346 us against 373-376 us), 4 for d = 32 (109 us with 8 against 105 us).
constexpr int waves_for(int64_t d) { return d == 32 || d % 32 != 0 ? kWaves : 8; }

// Wavefronts per workgroup for one launch: waves_for(d), except 4 for d = 64 and 128 when
// workgroups of 8 would leave fewer than two per CU (causal) or idle CUs. Causal work grows with
// the query block, and with that few workgroups the longest decides the time (1 x 16 x 4096 x 64:
// 16 heads x 16 query blocks of 256, 1 to 16 units of work, one workgroup per CU). With 4, twice
// as many half-size workgroups, two resident per CU, are issued paired (see AttnParams::paired),
// so each CU's pair sums to about the average.
int waves_used(int64_t d, int64_t lq, int64_t batch_count, bool causal, int cus) {
    const int w = waves_for(d);
    if (w == 4) {
        return 4;
    }
    const int64_t blocks = batch_count * ((lq + 32 * w - 1) / (32 * w));
    return blocks < (causal ? 2 : 1) * static_cast<int64_t>(cus) ? 4 : w;
}
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
    const float* q;
    const float* k;
    const float* v;
    float* out;
    const uint8_t* mask;
    int64_t lq, lk;
    int64_t q_rs, k_rs, v_rs, out_rs, mask_rs, mask_cs;
    int64_t batch[MFR_MAX_BATCH_DIMS];
    int64_t q_bs[MFR_MAX_BATCH_DIMS], k_bs[MFR_MAX_BATCH_DIMS], v_bs[MFR_MAX_BATCH_DIMS];
    int64_t out_bs[MFR_MAX_BATCH_DIMS], mask_bs[MFR_MAX_BATCH_DIMS];
    int64_t batch_count;
    int32_t batch_dims;
    int32_t causal;
    int32_t q_blocks;
    // Issue order of the query blocks: longest first, or (paired) the longer half longest first,
    // then the shorter half shortest first.
    int32_t paired;
    float scale;
};

// Which (batch entry, query block) workgroup blockIdx.x computes, and that entry's element
// offsets into q, k, v, out and the mask. Query blocks are issued longest first (the last ones of
// every batch entry), or, when paired, the longer half longest first and then the shorter half
// shortest first.
struct BlockWork {
    int64_t qb;
    int64_t off_q, off_k, off_v, off_o, off_m;
};

// The indices are below the workgroup count (under 2^31), so the decomposition runs in 32-bit
// unsigned arithmetic: a 64-bit division is a long scalar instruction sequence that every
// wavefront of the workgroup runs before its first load.
__device__ inline BlockWork block_work(const AttnParams& p) {
    const uint32_t bid = blockIdx.x;
    const uint32_t batch_count = static_cast<uint32_t>(p.batch_count);
    const uint32_t q_blocks = static_cast<uint32_t>(p.q_blocks);
    const uint32_t level = bid / batch_count;
    const uint32_t longer = (q_blocks + 1) / 2;
    BlockWork w{};
    w.qb = !p.paired || level < longer ? q_blocks - 1 - level : level - longer;
    uint32_t bi = bid - level * batch_count;
    for (int d = p.batch_dims - 1; d >= 0; --d) {
        const uint32_t extent = static_cast<uint32_t>(p.batch[d]);
        const int64_t idx = bi % extent;
        bi /= extent;
        w.off_q += idx * p.q_bs[d];
        w.off_k += idx * p.k_bs[d];
        w.off_v += idx * p.v_bs[d];
        w.off_o += idx * p.out_bs[d];
        w.off_m += idx * p.mask_bs[d];
    }
    return w;
}

// max / sum of the values in lanes l and l ^ 16 (rows16) or l and l ^ 32 (halves), in every lane,
// through the vector ALU's lane swaps (mfr::dev::swap_pair), not an LDS-crossbar permute and its
// wait on the softmax's critical path; every lane of a pair gets the same bits.
using mfr::dev::swap_pair;
__device__ inline float max_rows16(float x) {
    float a, b;
    swap_pair<false>(x, a, b);
    return fmaxf(a, b);
}
__device__ inline float max_halves(float x) {
    float a, b;
    swap_pair<true>(x, a, b);
    return fmaxf(a, b);
}
__device__ inline float sum_rows16(float x) {
    float a, b;
    swap_pair<false>(x, a, b);
    return a + b;
}
__device__ inline float sum_halves(float x) {
    float a, b;
    swap_pair<true>(x, a, b);
    return a + b;
}

// exp(x - m) through the hardware's 2^x (v_exp_f32, 1 ulp; results below 2^-126 may flush to
// zero, which is below the rounding of any row sum, whose largest term is exp(0) = 1). m is
// never -inf here (the caller substitutes 0), so x = -inf gives exp2(-inf) = 0 without a NaN.
__device__ inline float weight(float x, float m) {
    return __builtin_amdgcn_exp2f((x - m) * kLog2e);
}

// MASKED: a mask tensor is given (read for every score). Without it only the key count and the
// causal diagonal remove scores, and only blocks that reach past either are checked. WAVES
// wavefronts of 32 queries per workgroup; MIN_WAVES is the occupancy the compiler must allow
// (wavefronts per SIMD).
template <int D, int BK, bool MASKED, int WAVES = kWaves, int MIN_WAVES = 2>
__global__ __launch_bounds__(WAVES * 64, MIN_WAVES) void attention_kernel(AttnParams p) {
    constexpr int THREADS = WAVES * 64;
    constexpr int BLOCK_Q = WAVES * 32;
    constexpr int SUB = BK / 32; // 32-key sub-blocks per key block
    // d need not be a multiple of 32: the output side runs on DP = d rounded up to 32, whose V
    // rows past d load as zeros, so those output columns are zero and never stored.
    static_assert(D % 16 == 0, "d is a multiple of 16");
    constexpr int DP = (D + 31) / 32 * 32;
    constexpr int DB = DP / 32;  // 32-wide output column blocks
    constexpr int G = D / 8;     // depth groups of q . k
    constexpr int kStagePitch = DP + 4;
    using LoadK = SliceLoader<BK, D, true, 4, THREADS>;   // rows = keys, depth = d
    using LoadV = SliceLoader<DP, BK, false, 4, THREADS>; // rows = d (DP), depth = keys
    // Double-buffered K and V tiles; after the key loop the same memory stages the output.
    constexpr int kTileFloats = 2 * (LoadK::kFloats + LoadV::kFloats);
    constexpr int kStageFloats = WAVES * 32 * kStagePitch;
    __shared__ float smem[kTileFloats > kStageFloats ? kTileFloats : kStageFloats];
    auto lds_k = [&](int which) { return smem + which * LoadK::kFloats; };
    auto lds_v = [&](int which) { return smem + 2 * LoadK::kFloats + which * LoadV::kFloats; };

    // ---- which (batch entry, query block): the longest (last) query blocks first ----
    const BlockWork work = block_work(p);
    const int64_t qb = work.qb;
    const int64_t off_q = work.off_q, off_k = work.off_k, off_v = work.off_v,
                  off_o = work.off_o, off_m = work.off_m;

    const int lane = threadIdx.x % 64;
    // Uniform across the wavefront; read into a scalar register so that the branches on it
    // (active sub-blocks, edge blocks) are scalar branches.
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / 64));
    const int half = lane / 32;
    const int r32 = lane % 32;
    const int64_t q0 = qb * BLOCK_Q;
    const int64_t wq0 = q0 + wave * 32; // first query of this wavefront
    const int64_t query = wq0 + r32;    // this lane's query
    const bool wave_live = wq0 < p.lq;

    // q fragments: B operand of S^T = K Q^T, depth 8g + 4*half + s at step s of group g.
    float qf[G][4];
    {
        const float* qrow = p.q + off_q + query * p.q_rs + 4 * half;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (query < p.lq) {
                v = *reinterpret_cast<const float4*>(qrow + 8 * g);
            }
            qf[g][0] = v.x;
            qf[g][1] = v.y;
            qf[g][2] = v.z;
            qf[g][3] = v.w;
        }
    }
    const uint8_t* mask_row = nullptr;
    if constexpr (MASKED) {
        mask_row = p.mask + off_m + (query < p.lq ? query : 0) * p.mask_rs;
    }

    // Keys this workgroup needs: all of them, or (causal) up to its last query.
    int64_t k_end = p.lk;
    if (p.causal) {
        const int64_t last_query = (q0 + BLOCK_Q < p.lq ? q0 + BLOCK_Q : p.lq) - 1;
        k_end = last_query + 1 < k_end ? last_query + 1 : k_end;
    }
    const int64_t blocks = (k_end + BK - 1) / BK;

    float m_run = -INFINITY; // running maximum of this lane's query
    float l_run = 0.0f;      // this lane's share of the running sum (its 16 keys per sub-block)
    floatx16 oacc[DB];
#pragma unroll
    for (int b = 0; b < DB; ++b) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            oacc[b][e] = 0.0f;
        }
    }

    const float* k_base = p.k + off_k;
    const float* v_base = p.v + off_v;

    // Keys of block `blk` inside the matrix, and whether this wavefront needs the block at all
    // (uniform across the wavefront: causal attention skips blocks lying wholly above its
    // queries' diagonal). Inside a needed block every MFMA runs unconditionally (masking removes
    // what is not wanted), which keeps the accumulators in place.
    auto keys_in = [&](int64_t blk) {
        const int64_t left = p.lk - blk * BK;
        return left < BK ? static_cast<int>(left) : BK;
    };
    auto needed = [&](int64_t blk) { return wave_live && (!p.causal || blk * BK <= wq0 + 31); };

    // ---- S^T = K Q^T for one block, the sub-blocks' accumulator chains interleaved ----
    auto scores = [&](const float* sk, floatx16(&sacc)[SUB]) {
#pragma unroll
        for (int sb = 0; sb < SUB; ++sb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                sacc[sb][e] = 0.0f;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float kf[SUB][4];
#pragma unroll
            for (int sb = 0; sb < SUB; ++sb) {
                LoadK::fragment(sk, 32 * sb + r32, g, half, kf[sb]);
            }
#pragma unroll
            for (int st = 0; st < 4; ++st) {
#pragma unroll
                for (int sb = 0; sb < SUB; ++sb) {
                    sacc[sb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[sb][st], qf[g][st],
                                                                     sacc[sb], 0, 0, 0);
                }
            }
        }
    };

    // ---- scale, mask and the online softmax of the block starting at key k0: sacc becomes
    //      the weights exp(s - m) (per lane: query `query`, 16 keys per sub-block) ----
    auto softmax = [&](int64_t k0, floatx16(&sacc)[SUB]) {
        // Key of element e of sub-block sb, relative to k0: 32*sb + 8*(e/4) + e%4 + 4*half.
        // A block needs checking when it reaches past the last key or (causal) past the
        // wavefront's first query; both tests are uniform across the wavefront.
        const bool edge = k0 + BK > p.lk || (p.causal && k0 + BK - 1 > wq0);
        if (MASKED || edge) {
            const int64_t keys_left = p.lk - k0;
            const int64_t diag = query - k0; // causal keeps relative keys <= diag
            const int lim_k = static_cast<int>(keys_left < BK ? keys_left : BK) - 4 * half;
            const int lim_q = static_cast<int>(!p.causal || diag >= BK ? BK
                                               : diag < -1 ? -1
                                                           : diag) -
                              4 * half;
#pragma unroll
            for (int sb = 0; sb < SUB; ++sb) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int rel = 32 * sb + 8 * (e / 4) + e % 4; // minus 4*half (above)
                    bool keep = rel < lim_k && rel <= lim_q;
                    if constexpr (MASKED) {
                        if (keep) {
                            keep = mask_row[(k0 + rel + 4 * half) * p.mask_cs] != 0;
                        }
                    }
                    sacc[sb][e] = keep ? p.scale * sacc[sb][e] : -INFINITY;
                }
            }
        } else {
#pragma unroll
            for (int sb = 0; sb < SUB; ++sb) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    sacc[sb][e] = p.scale * sacc[sb][e];
                }
            }
        }
        float block_max = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < SUB; ++sb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                block_max = fmaxf(block_max, sacc[sb][e]);
            }
        }
        block_max = max_halves(block_max);
        const float m_new = fmaxf(m_run, block_max);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float rescale = weight(m_run, m_use); // exactly 1 where the maximum stayed
        m_run = m_new;
        l_run *= rescale;
#pragma unroll
        for (int b = 0; b < DB; ++b) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                oacc[b][e] *= rescale;
            }
        }
#pragma unroll
        for (int sb = 0; sb < SUB; ++sb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float w = weight(sacc[sb][e], m_use);
                sacc[sb][e] = w;
                l_run += w;
            }
        }
    };

    // ---- O^T += V^T P^T: P^T's fragments are the S^T accumulators themselves ----
    auto accumulate = [&](const float* sv, const floatx16(&sacc)[SUB]) {
#pragma unroll
        for (int sb = 0; sb < SUB; ++sb) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float vf[DB][4];
#pragma unroll
                for (int b = 0; b < DB; ++b) {
                    LoadV::fragment(sv, 32 * b + r32, 4 * sb + g, half, vf[b]);
                }
#pragma unroll
                for (int st = 0; st < 4; ++st) {
#pragma unroll
                    for (int b = 0; b < DB; ++b) {
                        oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            vf[b][st], sacc[sb][4 * g + st], oacc[b], 0, 0, 0);
                    }
                }
            }
        }
    };

    LoadK lk_;
    LoadV lv_;
    if (blocks > 0) {
        lk_.load(k_base, p.k_rs, 1, keys_in(0), D);
        lv_.load(v_base, 1, p.v_rs, D, keys_in(0));
        lk_.store(lds_k(0));
        lv_.store(lds_v(0));
        __syncthreads();
    }
    // One barrier per block: the next block's tiles are loaded into registers while this one is
    // computed, then written to the other buffers. (A software-pipelined form, K one block
    // ahead so the next scores' MFMAs overlap this block's softmax, gave the same bits but ran
    // 198-202 us against 183-186 us at configs[4].)
    for (int64_t kb = 0; kb < blocks; ++kb) {
        const int cur = static_cast<int>(kb & 1);
        const bool more = kb + 1 < blocks;
        if (more) {
            lk_.load(k_base + (kb + 1) * BK * p.k_rs, p.k_rs, 1, keys_in(kb + 1), D);
            lv_.load(v_base + (kb + 1) * BK * p.v_rs, 1, p.v_rs, D, keys_in(kb + 1));
        }
        if (needed(kb)) {
            floatx16 sacc[SUB];
            scores(lds_k(cur), sacc);
            softmax(kb * BK, sacc);
            accumulate(lds_v(cur), sacc);
        }
        if (more) {
            lk_.store(lds_k(cur ^ 1));
            lv_.store(lds_v(cur ^ 1));
        }
        __syncthreads();
    }

    // ---- normalise, stage [32 queries][D] per wavefront in LDS, store 16-byte rows ----
    const float l_total = sum_halves(l_run);
    // A row whose every key was removed has l_total == 0 and gives zeros; a NaN score makes
    // l_total NaN and so the whole row.
    const float inv = l_total == 0.0f ? 0.0f : 1.0f / l_total;
    float* stage = smem + wave * 32 * kStagePitch;
    __syncthreads();
#pragma unroll
    for (int b = 0; b < DB; ++b) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int col = 32 * b + 8 * (e / 4) + 4 * half + e % 4;
            stage[r32 * kStagePitch + col] = oacc[b][e] * inv;
        }
    }
    __syncthreads();
    float* out_base = p.out + off_o;
    constexpr int kRowUnits = D / 4;
#pragma unroll
    for (int i = 0; i < 32 * kRowUnits / 64; ++i) {
        const int u = lane + 64 * i;
        const int row = u / kRowUnits;
        const int c4 = u % kRowUnits;
        const int64_t qrow = wq0 + row;
        if (qrow < p.lq) {
            *reinterpret_cast<float4*>(out_base + qrow * p.out_rs + 4 * c4) =
                *reinterpret_cast<const float4*>(stage + row * kStagePitch + 4 * c4);
        }
    }
}

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Wavefronts per workgroup of attention16_kernel: 8 (128 queries, two workgroups per CU, 4
// wavefronts per SIMD), so one workgroup's prologue, diagonal blocks and output store overlap the
// other's key loop: configs[4] 173.9 against 176.2 us with 16 (256 queries, one per CU) on one box.
// (Before the K/V buffer loads took the kernel from 120 to 100 registers, 16 measured faster:
// 162.9 against 165.2 us.)
constexpr int kWaves16 = 8;

// The same op with 16 queries per wavefront on v_mfma_f32_16x16x4_f32 (4x4 accumulators per
// lane per 16x16 block): a wavefront holds 16 scores, 16 output values and D/4 query values per
// lane, a third of the 32-query form's registers, so 4 wavefronts fit on a SIMD.
//   - S^T = K Q^T per 16-key block j: lane l supplies K(16j + l%16, d) and Q(l%16, d) at depth
//     d = 16a + 4(l/16) + b on step (a, b) (both operands use that permutation, so the sum is
//     unchanged), which makes each lane's K values for 4 steps one 16-byte LDS read. Lane l then
//     holds the scores of query l%16 with keys 16j + 4(l/16) + r, r = 0..3: the four lanes
//     l%16 + 16g share a query, and its maximum and sum take two exchanges.
//   - O^T += V^T P^T over key steps (j, r): lane l's B value is its own score register
//     sacc[j][r] (query l%16, key 16j + 4(l/16) + r), and its A value V(key, 16c + l%16), read
//     from a transposed V tile [d][BK+4] as one 16-byte read per 4 steps.
//   - K tiles come by direct-to-LDS buffer loads into [keys][D], their 16-byte pieces swizzled
//     (piece c of key r at c ^ (r & 15)) in place of padding; V tiles are written transposed
//     (each thread loads 4 adjacent d of one key and stores them down a column; adjacent lanes
//     take adjacent keys, so the stores hit distinct banks). Both are double-buffered with one
//     barrier per key block, the key loop unrolled by two so each half names its K buffers.
//     (V^T by 4-byte direct loads, each a 64-key gather, measured 182 against 174 us.)
template <int D, int BK, bool MASKED, int WAVES>
__global__ __launch_bounds__(WAVES * 64, 4) void attention16_kernel(AttnParams p) {
    constexpr int THREADS = WAVES * 64;
    constexpr int BLOCK_Q = WAVES * 16;
    constexpr int KB = BK / 16;  // 16-key blocks per key block
    constexpr int DB = D / 16;   // 16-wide output column blocks; 16-deep groups of q . k
    constexpr int VP = BK + 4;   // V^T tile pitch
    constexpr int kVFloats = D * VP;
    constexpr int kStagePitch = D + 4;
    constexpr int kStageFloats = BLOCK_Q * kStagePitch;
    constexpr int kQuads = BK * (D / 4);                              // 16-byte pieces per V tile
    constexpr int kLoads = (kQuads + THREADS - 1) / THREADS;          // per thread per tile
    static_assert(D == 64 && BK == 64, "the swizzled K tile takes 64 keys of 16 pieces");
    constexpr int kKFloats = BK * D;
    constexpr int kKInstr = kKFloats / 256; // 1 KiB wave-instructions per K tile
    constexpr int kKPerWave = kKInstr / WAVES;
    static_assert(kKInstr % WAVES == 0, "K tile instructions per wavefront");
    constexpr int kVTiles = 2 * kVFloats > kStageFloats ? 2 * kVFloats : kStageFloats;
    // One LDS object per K buffer: the compiler then sees that the direct-to-LDS copy into one
    // does not write the one the score MFMAs read, and does not wait for the copy to land before
    // those reads. The output stage reuses the V tiles.
    __shared__ __align__(16) float k_tile0[kKFloats];
    __shared__ __align__(16) float k_tile1[kKFloats];
    __shared__ __align__(16) float v_tiles[kVTiles];
    auto lds_v = [&](int which) { return v_tiles + which * kVFloats; };

    const BlockWork work = block_work(p);
    const int64_t qb = work.qb;
    const int64_t off_q = work.off_q, off_k = work.off_k, off_v = work.off_v,
                  off_o = work.off_o, off_m = work.off_m;

    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / 64));
    const int g = lane / 16;   // which 4 of each 16 keys (and depths) this lane takes
    const int col = lane % 16; // this lane's query within the wavefront's 16
    const int64_t q0 = qb * BLOCK_Q;
    const int64_t wq0 = q0 + wave * 16;
    const int64_t query = wq0 + col;
    const bool wave_live = wq0 < p.lq;

    // q is held pre-multiplied by scale * log2(e), so the scores come out of the MFMAs already
    // scaled and in base-2 units: the softmax's weights are then exp2(s - m) with no multiply
    // per score.
    float qf[DB][4];
    {
        const float* qrow = p.q + off_q + query * p.q_rs + 4 * g;
        const float to_log2 = p.scale * kLog2e;
#pragma unroll
        for (int a = 0; a < DB; ++a) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (query < p.lq) {
                v = *reinterpret_cast<const float4*>(qrow + 16 * a);
            }
            qf[a][0] = v.x * to_log2;
            qf[a][1] = v.y * to_log2;
            qf[a][2] = v.z * to_log2;
            qf[a][3] = v.w * to_log2;
        }
    }
    const uint8_t* mask_row = nullptr;
    if constexpr (MASKED) {
        mask_row = p.mask + off_m + (query < p.lq ? query : 0) * p.mask_rs;
    }

    int64_t k_end = p.lk;
    if (p.causal) {
        const int64_t last_query = (q0 + BLOCK_Q < p.lq ? q0 + BLOCK_Q : p.lq) - 1;
        k_end = last_query + 1 < k_end ? last_query + 1 : k_end;
    }
    const int64_t blocks = (k_end + BK - 1) / BK;

    float m_run = -INFINITY;
    float l_run = 0.0f;
    floatx4 oacc[DB];
#pragma unroll
    for (int c = 0; c < DB; ++c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            oacc[c][r] = 0.0f;
        }
    }

    const float* k_base = p.k + off_k;
    const float* v_base = p.v + off_v;
    auto keys_in = [&](int64_t blk) {
        const int64_t left = p.lk - blk * BK;
        return left < BK ? static_cast<int>(left) : BK;
    };
    auto needed = [&](int64_t blk) { return wave_live && (!p.causal || blk * BK <= wq0 + 15); };

    // Tile loads: piece u of V is (key u % BK, depths 4(u / BK)..+3). K and V come by buffer
    // loads: the block's first key row is the resource's base and its record count ends after
    // the block's last key, so pieces of keys past the end read as zeros with no per-lane test,
    // and a lane's byte offset within a tile is a register fixed for the whole key loop (the
    // host keeps BK rows under 2^30 bytes). Loads through a per-block address register made the
    // compiler wait for them before the next LDS reads.
    float4 vr[kLoads];
    uint32_t v_off[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int u = static_cast<int>(threadIdx.x) + i * THREADS;
        const int vkey = u % BK, vq = u / BK;
        v_off[i] = u < kQuads ? static_cast<uint32_t>((vkey * p.v_rs + 4 * vq) * 4) : 0x80000000u;
    }
    auto tile_load = [](const float* rows, int64_t row_stride, int keys, uint32_t offset) {
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(rows), 0, static_cast<int>(keys * row_stride * 4), 0x00020000);
        const u32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(offset),
                                                                0, 0);
        return make_float4(__uint_as_float(raw.x), __uint_as_float(raw.y),
                           __uint_as_float(raw.z), __uint_as_float(raw.w));
    };
    auto load_v = [&](int64_t blk) {
        const int keys = keys_in(blk);
        const float* vb = v_base + blk * BK * p.v_rs;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            vr[i] = tile_load(vb, p.v_rs, keys, v_off[i]);
        }
    };
    auto store_v = [&](int which) {
        float* sv = lds_v(which);
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int u = static_cast<int>(threadIdx.x) + i * THREADS;
            if (u < kQuads) {
                const int vkey = u % BK, vq = u / BK;
                sv[(4 * vq + 0) * VP + vkey] = vr[i].x;
                sv[(4 * vq + 1) * VP + vkey] = vr[i].y;
                sv[(4 * vq + 2) * VP + vkey] = vr[i].z;
                sv[(4 * vq + 3) * VP + vkey] = vr[i].w;
            }
        }
    };
    // K by direct-to-LDS buffer loads into [keys][D] with no padding: instruction i of a tile
    // (keys 4i..4i+3) writes lane L's 16 bytes at L * 16, key 4i + L/16, physical piece L % 16,
    // which holds logical piece (L % 16) ^ (key & 15). A lane reading key 16j + col, piece c,
    // finds it at piece c ^ col, so 16 lanes with 16 keys read 16 different pieces. (Loaded into
    // registers and stored to a padded tile, config 5 measured 1-2 % slower.)
    uint32_t kd_off[kKPerWave];
#pragma unroll
    for (int j = 0; j < kKPerWave; ++j) {
        const int key = 4 * (wave * kKPerWave + j) + lane / 16;
        const int piece = (lane % 16) ^ (key & 15);
        kd_off[j] = static_cast<uint32_t>((key * p.k_rs + 4 * piece) * 4);
    }
    auto direct_k = [&](int64_t blk, float* dst) {
        const int keys = keys_in(blk);
        const float* kb = k_base + blk * BK * p.k_rs;
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(kb), 0, static_cast<int>(keys * p.k_rs * 4), 0x00020000);
#pragma unroll
        for (int j = 0; j < kKPerWave; ++j) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst + (wave * kKPerWave + j) * 256, 16,
                                                     static_cast<int>(kd_off[j]), 0, 0, 0);
        }
    };

    auto scores = [&](const float* sk, floatx4(&sacc)[KB]) {
#pragma unroll
        for (int j = 0; j < KB; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sacc[j][r] = 0.0f;
            }
        }
#pragma unroll
        for (int a = 0; a < DB; ++a) {
            float4 kf[KB];
#pragma unroll
            for (int j = 0; j < KB; ++j) {
                kf[j] = *reinterpret_cast<const float4*>(sk + (16 * j + col) * D +
                                                         4 * ((4 * a + g) ^ col));
            }
#pragma unroll
            for (int b = 0; b < 4; ++b) {
#pragma unroll
                for (int j = 0; j < KB; ++j) {
                    const float kv = b == 0 ? kf[j].x : b == 1 ? kf[j].y : b == 2 ? kf[j].z : kf[j].w;
                    sacc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv, qf[a][b], sacc[j], 0, 0, 0);
                }
            }
        }
    };

    // Scale, mask and the online softmax of the block at key k0 (element r of block j: relative
    // key 16j + 4g + r).
    auto softmax = [&](int64_t k0, floatx4(&sacc)[KB]) {
        const bool edge = k0 + BK > p.lk || (p.causal && k0 + BK - 1 > wq0);
        if (MASKED || edge) {
            // In 32-bit lane arithmetic (the 64-bit forms cost registers the key loop lacks):
            // the wavefront's first query's diagonal offset, clamped to [-32, BK] while uniform,
            // then this lane's query added (col < 16 keeps both clamps' outcomes).
            const int64_t keys_left = p.lk - k0;
            const int64_t first_diag = wq0 - k0;
            const int base = static_cast<int>(first_diag < -32 ? -32
                                              : first_diag > BK ? BK
                                                                : first_diag);
            const int diag = base + col;
            const int lim_k = static_cast<int>(keys_left < BK ? keys_left : BK) - 4 * g;
            const int lim_q = (!p.causal || diag >= BK ? BK : diag < -1 ? -1 : diag) - 4 * g;
#pragma unroll
            for (int j = 0; j < KB; ++j) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rel = 16 * j + r; // minus 4g (above)
                    bool keep = rel < lim_k && rel <= lim_q;
                    if constexpr (MASKED) {
                        if (keep) {
                            keep = mask_row[(k0 + rel + 4 * g) * p.mask_cs] != 0;
                        }
                    }
                    sacc[j][r] = keep ? sacc[j][r] : -INFINITY;
                }
            }
        }
        float block_max = -INFINITY;
#pragma unroll
        for (int j = 0; j < KB; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                block_max = fmaxf(block_max, sacc[j][r]);
            }
        }
        block_max = max_halves(max_rows16(block_max));
        const float m_new = fmaxf(m_run, block_max);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        // The rescale is 1 for every lane whose maximum stayed (most blocks past the first few):
        // skipped when that holds for the whole wavefront.
        if (__ballot(m_new != m_run) != 0) {
            const float rescale = __builtin_amdgcn_exp2f(m_run - m_use);
            l_run *= rescale;
#pragma unroll
            for (int c = 0; c < DB; ++c) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    oacc[c][r] *= rescale;
                }
            }
        }
        m_run = m_new;
#pragma unroll
        for (int j = 0; j < KB; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float w = __builtin_amdgcn_exp2f(sacc[j][r] - m_use);
                sacc[j][r] = w;
                l_run += w;
            }
        }
    };

    auto accumulate = [&](const float* sv, const floatx4(&sacc)[KB]) {
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            float4 vf[DB];
#pragma unroll
            for (int c = 0; c < DB; ++c) {
                vf[c] = *reinterpret_cast<const float4*>(sv + (16 * c + col) * VP + 16 * j + 4 * g);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma unroll
                for (int c = 0; c < DB; ++c) {
                    const float vv = r == 0 ? vf[c].x : r == 1 ? vf[c].y : r == 2 ? vf[c].z : vf[c].w;
                    oacc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv, sacc[j][r], oacc[c], 0, 0, 0);
                }
            }
        }
    };

    // One key block: the next block's K copy (direct to LDS) and V loads are issued first, the
    // V tile stored after this block's products, and the copy waited for before the barrier.
    auto step = [&](int64_t kb, float* k_cur, float* k_next, int cur) {
        const bool more = kb + 1 < blocks;
        if (more) {
            direct_k(kb + 1, k_next);
            load_v(kb + 1);
        }
        if (needed(kb)) {
            floatx4 sacc[KB];
            scores(k_cur, sacc);
            softmax(kb * BK, sacc);
            accumulate(lds_v(cur), sacc);
        }
        if (more) {
            store_v(cur ^ 1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };
    if (blocks > 0) {
        direct_k(0, k_tile0);
        load_v(0);
        store_v(0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    for (int64_t kb = 0; kb < blocks; kb += 2) {
        step(kb, k_tile0, k_tile1, 0);
        if (kb + 1 < blocks) {
            step(kb + 1, k_tile1, k_tile0, 1);
        }
    }

    // ---- normalise, stage [16 queries][D] per wavefront in LDS, store 16-byte rows ----
    const float l_total = sum_halves(sum_rows16(l_run));
    const float inv = l_total == 0.0f ? 0.0f : 1.0f / l_total;
    float* stage = v_tiles + wave * 16 * kStagePitch;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < DB; ++c) {
        *reinterpret_cast<float4*>(stage + col * kStagePitch + 16 * c + 4 * g) =
            make_float4(oacc[c][0] * inv, oacc[c][1] * inv, oacc[c][2] * inv, oacc[c][3] * inv);
    }
    __syncthreads();
    float* out_base = p.out + off_o;
    constexpr int kRowUnits = D / 4;
#pragma unroll
    for (int i = 0; i < 16 * kRowUnits / 64; ++i) {
        const int u = lane + 64 * i;
        const int row = u / kRowUnits;
        const int c4 = u % kRowUnits;
        const int64_t qrow = wq0 + row;
        if (qrow < p.lq) {
            *reinterpret_cast<float4*>(out_base + qrow * p.out_rs + 4 * c4) =
                *reinterpret_cast<const float4*>(stage + row * kStagePitch + 4 * c4);
        }
    }
}

template <bool MASKED>
void launch(int64_t d, int waves, const AttnParams& p, unsigned grid, hipStream_t st) {
    switch (d) {
    case 32:
        // 3 wavefronts per SIMD where the registers allow it (148 VGPRs without a mask):
        // 102.9 us against 105.3 us with 2.
        attention_kernel<32, 64, MASKED, waves_for(32), MASKED ? 2 : 3>
            <<<grid, waves_for(32) * 64, 0, st>>>(p);
        break;
    case 64:
        if (waves == 4) {
            attention_kernel<64, 64, MASKED, 4><<<grid, 4 * 64, 0, st>>>(p);
        } else {
            attention_kernel<64, 64, MASKED, waves_for(64)><<<grid, waves_for(64) * 64, 0, st>>>(
                p);
        }
        break;
    case 16:
        attention_kernel<16, 64, MASKED, 4><<<grid, 4 * 64, 0, st>>>(p);
        break;
    case 48:
        attention_kernel<48, 64, MASKED, 4><<<grid, 4 * 64, 0, st>>>(p);
        break;
    case 80:
        attention_kernel<80, 64, MASKED, 4><<<grid, 4 * 64, 0, st>>>(p);
        break;
    case 112:
        attention_kernel<112, 64, MASKED, 4><<<grid, 4 * 64, 0, st>>>(p);
        break;
    case 96:
        if (waves == 4) {
            attention_kernel<96, 32, MASKED, 4><<<grid, 4 * 64, 0, st>>>(p);
        } else {
            attention_kernel<96, 64, MASKED, waves_for(96)><<<grid, waves_for(96) * 64, 0, st>>>(
                p);
        }
        break;
    default:
        if (waves == 4) {
            attention_kernel<128, 32, MASKED, 4><<<grid, 4 * 64, 0, st>>>(p);
        } else {
            attention_kernel<128, 32, MASKED, waves_for(128)>
                <<<grid, waves_for(128) * 64, 0, st>>>(p);
        }
        break;
    }
}

bool aligned_rows(const void* base, int64_t row_stride, const int64_t* bs, int dims) {
    if (!mfr::aligned16(base) || row_stride % 4 != 0) {
        return false;
    }
    for (int d = 0; d < dims; ++d) {
        if (bs[d] % 4 != 0) {
            return false;
        }
    }
    return true;
}

void run_attention(mfr_stream& s, const mfr_attention_desc& d) {
    using mfr::require;
    require(d.lq >= 0 && d.lk >= 0 && d.d >= 0, "attention: negative dimension");
    require(d.batch_dims >= 0 && d.batch_dims <= MFR_MAX_BATCH_DIMS,
            "attention: batch_dims out of range");
    int64_t batch_count = 1;
    for (int i = 0; i < d.batch_dims; ++i) {
        require(d.batch[i] >= 0, "attention: negative batch size");
        batch_count *= d.batch[i];
    }
    if (d.lq == 0 || batch_count == 0) {
        return;
    }
    if (d.d <= 0 || d.d > 128 || d.d % 16 != 0) {
        throw mfr::Error(MFR_E_UNSUPPORTED,
                         "attention: fused kernel takes d = 16, 32, ..., 128 (a multiple of 16)");
    }
    require(d.q != nullptr && d.out != nullptr, "attention: null q or out");
    require(d.lk == 0 || (d.k != nullptr && d.v != nullptr), "attention: null k or v");
    require(d.q_rs >= d.d && d.out_rs >= d.d, "attention: row stride smaller than d");
    const bool aligned =
        aligned_rows(d.q, d.q_rs, d.q_bs, d.batch_dims) &&
        aligned_rows(d.out, d.out_rs, d.out_bs, d.batch_dims) &&
        (d.lk == 0 || (aligned_rows(d.k, d.k_rs, d.k_bs, d.batch_dims) &&
                       aligned_rows(d.v, d.v_rs, d.v_bs, d.batch_dims)));
    if (!aligned) {
        throw mfr::Error(MFR_E_UNSUPPORTED,
                         "attention: fused kernel needs 16-byte aligned rows and strides");
    }
    AttnParams p{};
    p.q = d.q;
    p.k = d.k;
    p.v = d.v;
    p.out = d.out;
    p.mask = d.mask;
    p.lq = d.lq;
    p.lk = d.lk;
    p.q_rs = d.q_rs;
    p.k_rs = d.k_rs;
    p.v_rs = d.v_rs;
    p.out_rs = d.out_rs;
    p.mask_rs = d.mask != nullptr ? d.mask_rs : 0;
    p.mask_cs = d.mask != nullptr ? d.mask_cs : 0;
    p.batch_dims = d.batch_dims;
    for (int i = 0; i < d.batch_dims; ++i) {
        p.batch[i] = d.batch[i];
        p.q_bs[i] = d.q_bs[i];
        p.k_bs[i] = d.k_bs[i];
        p.v_bs[i] = d.v_bs[i];
        p.out_bs[i] = d.out_bs[i];
        p.mask_bs[i] = d.mask != nullptr ? d.mask_bs[i] : 0;
    }
    p.batch_count = batch_count;
    p.causal = d.causal != 0;
    p.scale = d.scale != 0.0f ? d.scale
                              : static_cast<float>(1.0 / std::sqrt(static_cast<double>(d.d)));
    const int waves = waves_used(d.d, d.lq, batch_count, d.causal != 0, s.compute_units);
    // d = 64, causal, no mask, a grid of 8-wavefront workgroups: the 16-query kernel, whose
    // last diagonal key blocks keep every SIMD busy (configs[4]: 163.6 against 170.0 us).
    // Non-causal it measured 291 against 288 us, at d = 32 96.9 against 93.5 us (causal) and
    // 169.6 against 159.8 us, and its masked form spills; those keep the 32-query kernel.
    const bool use16 = d.d == 64 && d.causal != 0 && d.mask == nullptr && waves == waves_for(64) &&
                       d.k_rs < (int64_t{1} << 22) && d.v_rs < (int64_t{1} << 22);
    const int64_t block_q = use16 ? 16 * kWaves16 : 32 * waves; // queries per workgroup
    const int64_t q_blocks = (d.lq + block_q - 1) / block_q;
    const int64_t blocks = q_blocks * batch_count;
    require(blocks < (int64_t{1} << 31), "attention: problem too large for one launch");
    p.q_blocks = static_cast<int32_t>(q_blocks);
    // Every workgroup resident at once (two per CU): the CU holding the j-th issued also holds
    // the (j + CUs)-th, so pair long with short. Otherwise CUs take the next as they free up,
    // and longest first balances.
    p.paired = p.causal && waves == 4 && waves_for(d.d) == 8 && blocks <= 2 * s.compute_units;
    const unsigned grid = static_cast<unsigned>(blocks);
    if (use16) {
        attention16_kernel<64, 64, false, kWaves16><<<grid, kWaves16 * 64, 0, s.stream>>>(p);
    } else if (d.mask != nullptr) {
        launch<true>(d.d, waves, p, grid, s.stream);
    } else {
        launch<false>(d.d, waves, p, grid, s.stream);
    }
    mfr::check_launch("attention_kernel");
}

} // namespace

extern "C" int mfr_attention(mfr_stream_t stream, const mfr_attention_desc* desc) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(desc != nullptr, "attention: null descriptor");
        run_attention(s, *desc);
    });
}
