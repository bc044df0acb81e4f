// tsp_spmm_bm64.hip -- the 64-row instantiations of spmm_kernel (tsp_spmm.hpp):
// the (chunk width, pipeline depth) pairs of the dense A format, plus the
// panel-synchronised dense sweep.
#include "tsp_spmm.hpp"

namespace tsp {

const void *select_kernel_bm64(int prec, int w, int s, bool packed, bool lane_idx, bool sync, bool pair)
{
    if (pair) return nullptr;   // 64-row fp16 tiles are 32 wide already (K = 32)
#define TSP_K(Wv, Sv, PKv, LIv, SYv)                                                  \
    if (w == Wv && s == Sv && packed == PKv && lane_idx == LIv && sync == SYv) \
        return pick_kernel<64, Wv, Sv, PKv, LIv, SYv>(prec);
#define X(Wv, Sv) TSP_K(Wv, Sv, false, false, false)
    X(32, 1) X(32, 2) X(32, 3) X(64, 1) X(64, 2) X(64, 3)
#undef X
#define X(Wv, Sv) TSP_K(Wv, Sv, false, false, true)
    X(64, 1) X(64, 2)
#undef X
#undef TSP_K
    return nullptr;
}

}  // namespace tsp
