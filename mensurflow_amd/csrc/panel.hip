// The panel path's launch (panel_kernel.hpp holds the design), in a translation unit of its own.
#include "panel_kernel.hpp"

namespace mfr::gemm {

namespace {

// The kernel for depth groups KG with non-temporal stores or not, and the full epilogue (beta *
// C0, bias) or alpha alone.
template <int KG>
void launch_depth(bool nt, bool full, unsigned grid, const PanelParams& pp, hipStream_t stream) {
    if (nt && full) {
        sgemm_panel_kernel<KG, true, true><<<grid, kPanelThreads, 0, stream>>>(pp);
    } else if (nt) {
        sgemm_panel_kernel<KG, true, false><<<grid, kPanelThreads, 0, stream>>>(pp);
    } else if (full) {
        sgemm_panel_kernel<KG, false, true><<<grid, kPanelThreads, 0, stream>>>(pp);
    } else {
        sgemm_panel_kernel<KG, false, false><<<grid, kPanelThreads, 0, stream>>>(pp);
    }
}

} // namespace

// The panel path on q: row panels of kPanelRows, column tiles of kPanelCols, and the tiles of
// each panel cut into ranges (workgroups of their own) until the grid holds at least two
// workgroups per CU. nt: non-temporal stores.
void launch_panel(const GemmParams& q, bool nt, int cus, hipStream_t stream) {
    PanelParams pp{};
    pp.g = q;
    pp.g.splits = 1;
    pp.g.partial = nullptr;
    const int64_t panels = (q.m + kPanelRows - 1) / kPanelRows;
    const int64_t nblocks = (q.n + kPanelCols - 1) / kPanelCols;
    const int64_t owners = panels * q.batch_count;
    int64_t chunks = (2 * static_cast<int64_t>(cus) + owners - 1) / owners;
    chunks = chunks < 1 ? 1 : chunks > nblocks ? nblocks : chunks;
    const int64_t per_chunk = (nblocks + chunks - 1) / chunks;
    chunks = (nblocks + per_chunk - 1) / per_chunk;
    const int64_t blocks = owners * chunks;
    mfr::require(blocks < (int64_t{1} << 31) && nblocks < (int64_t{1} << 30),
                 "sgemm: problem too large for one launch");
    pp.panels = static_cast<int32_t>(panels);
    pp.nblocks = static_cast<int32_t>(nblocks);
    pp.chunks = static_cast<int32_t>(chunks);
    pp.per_chunk = static_cast<int32_t>(per_chunk);
    const unsigned grid = static_cast<unsigned>(blocks);
    const bool full = (q.c0 != nullptr && q.beta != 0.0f) || q.bias != nullptr;
    if (q.k <= 16) {
        launch_depth<2>(nt, full, grid, pp, stream);
    } else if (q.k <= 32) {
        launch_depth<4>(nt, full, grid, pp, stream);
    } else {
        launch_depth<8>(nt, full, grid, pp, stream);
    }
}

} // namespace mfr::gemm
