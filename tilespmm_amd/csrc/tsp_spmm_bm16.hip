// tsp_spmm_bm16.hip -- the 16-row instantiations of spmm_kernel (tsp_spmm.hpp):
// the (chunk width, pipeline depth) pairs of the dense A format and of the
// packed format, each with scalar or lane-loaded column indices (dense: at
// chunks of up to 128 columns), plus the
// panel-synchronised dense sweep, and the fp16 tile-pair forms of each.
#include "tsp_spmm.hpp"

namespace tsp {

const void *select_kernel_bm16(int prec, int w, int s, bool packed, bool lane_idx, bool sync, bool pair)
{
    if (pair) {
        // tile pairs (fp16): 64- and 128-column chunks
#define TSP_P(Wv, Sv, PKv, LIv, SYv)                                                  \
    if (w == Wv && s == Sv && packed == PKv && lane_idx == LIv && sync == SYv) \
        return pick_pair_kernel<16, Wv, Sv, PKv, LIv, SYv>(prec);
#define X(Wv, Sv) TSP_P(Wv, Sv, false, false, false) TSP_P(Wv, Sv, false, false, true)
        X(64, 1) X(64, 2) X(128, 1) X(128, 2)
#undef X
#define X(Wv, Sv) TSP_P(Wv, Sv, true, false, false) TSP_P(Wv, Sv, true, true, false)
        X(64, 1) X(64, 2) X(64, 3) X(128, 1) X(128, 2) X(128, 3)
#undef X
#undef TSP_P
        return nullptr;
    }
#define TSP_K(Wv, Sv, PKv, LIv, SYv)                                                  \
    if (w == Wv && s == Sv && packed == PKv && lane_idx == LIv && sync == SYv) \
        return pick_kernel<16, Wv, Sv, PKv, LIv, SYv>(prec);
#define X(Wv, Sv) TSP_K(Wv, Sv, false, false, false)
    X(32, 1) X(32, 2) X(32, 3) X(64, 1) X(64, 2) X(64, 3) X(128, 1) X(128, 2) X(128, 3) X(256, 1) X(256, 2)
#undef X
    // dense tiles with lane-loaded column indices (chunks of up to 128 columns)
#define X(Wv, Sv) TSP_K(Wv, Sv, false, true, false)
    X(32, 1) X(32, 2) X(32, 3) X(64, 1) X(64, 2) X(64, 3) X(128, 1) X(128, 2) X(128, 3)
#undef X
#define X(Wv, Sv) TSP_K(Wv, Sv, true, false, false) TSP_K(Wv, Sv, true, true, false)
    X(32, 1) X(32, 2) X(32, 3) X(64, 1) X(64, 2) X(64, 3) X(128, 1) X(128, 2) X(128, 3) X(256, 1) X(256, 2)
#undef X
#define X(Wv, Sv) TSP_K(Wv, Sv, false, false, true)
    X(64, 1) X(64, 2) X(128, 1) X(128, 2) X(256, 1) X(256, 2)
#undef X
#undef TSP_K
    return nullptr;
}

}  // namespace tsp
