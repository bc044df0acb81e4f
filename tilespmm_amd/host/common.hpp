// common.hpp -- small helpers shared by the host library translation units.
#pragma once
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/tilespmm.h"

namespace tsph {

// IEEE binary16 <-> binary32 with the CPU's F16C unit (round to nearest even).
inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
inline uint16_t f2h(float f) { return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

// Round binary32 to tf32 (10 explicit mantissa bits), nearest even; inf/nan kept.
inline float round_tf32(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7f800000u) != 0x7f800000u) x = (x + 0xfffu + ((x >> 13) & 1u)) & 0xffffe000u;
    memcpy(&f, &x, 4);
    return f;
}

inline size_t val_size(int prec) { return prec == TSP_PREC_FP16 ? 2 : 4; }

template <typename T>
inline T *alloc_n(size_t n)
{
    return (T *)malloc(sizeof(T) * (n ? n : 1));
}

}  // namespace tsph
