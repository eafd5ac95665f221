// quant_xq's group step, shared by the kernels that quantize activations on their way out (quant.hip, attn.hip).
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

#include "xlane.h"
#include "../../include/strata_hip.h"

namespace strata {

// The quantization of 8 consecutive values v (positions i..i + 7 of a row; lanes past n hold zeros) by a group of 32
// lanes covering 256 values, as quant_xq does: the int8 values into q (the row's base) and one scale per 32 values into
// qd (the row's base). Every lane of the group takes part (the block maximum is a cross-lane reduction).
__device__ __forceinline__ void quant8_group(const float (&v)[8], int i, bool live, int mode, int8_t* q, float* qd) {
    float d, mul;
    if (mode == STRATA_NUM_Q8K) {
        // Candidate: the first value of largest magnitude among this lane's 8, then across the 32 lanes (lowest index).
        float bv = v[0];
        int bi = i;
#pragma unroll
        for (int j = 1; j < 8; j++) if (fabsf(v[j]) > fabsf(bv)) { bv = v[j]; bi = i + j; }
        // the first value of largest magnitude over the 32 lanes: the choice is unique, so the pairing of the
        // exchange steps does not matter
        auto step = [&](auto S) __attribute__((always_inline)) {
            constexpr int st = decltype(S)::value;
            const float ov = xl32f<st>(bv);
            const int oi = xl32<st>(bi);
            if (fabsf(ov) > fabsf(bv) || (fabsf(ov) == fabsf(bv) && oi < bi)) { bv = ov; bi = oi; }
        };
        step(std::integral_constant<int, 0>{});
        step(std::integral_constant<int, 1>{});
        step(std::integral_constant<int, 2>{});
        step(std::integral_constant<int, 3>{});
        step(std::integral_constant<int, 4>{});
        float is = bv != 0.0f ? -127.0f / bv : 0.0f;
        d = bv != 0.0f ? 1.0f / is : 0.0f;
        mul = is;
    } else {
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(v[j]));
        mx = fmaxf(mx, xl32f<0>(mx));
        mx = fmaxf(mx, xl32f<1>(mx));
        d = mx / 127.0f;
        mul = mx > 0.0f ? 127.0f / mx : 0.0f;
    }
    if (!live) return;
    uint32_t w[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float r = __builtin_rintf(mul * v[j]);
        int qq = (int)fminf(r, 127.0f);
        w[j >> 2] |= (uint32_t)(qq & 255) << (8 * (j & 3));
    }
    *(uint2*)(q + i) = make_uint2(w[0], w[1]);
    if ((threadIdx.x & 3) == 0) qd[i / 32] = d;
}

}  // namespace strata
