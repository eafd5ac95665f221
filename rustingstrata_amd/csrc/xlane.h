// Cross-lane exchanges for reductions within 32-lane groups, without the LDS round trip of a lane permute where DPP
// reaches: step 0 pairs lane ^ 1, step 1 lane ^ 2 (quad permutes), step 2 mirrors within 8 lanes, step 3 within 16
// (row mirrors), step 4 pairs lane ^ 16 (ds_swizzle, bit mode). Each step combines two disjoint halves of the
// previous steps' groups, so an associative and commutative reduction over steps 0..4 leaves every lane of the 32
// with the same result as an xor butterfly.
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

namespace strata {

template <int STEP>
__device__ __forceinline__ int xl32(int v) {
    if constexpr (STEP == 0) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    else if constexpr (STEP == 1) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    else if constexpr (STEP == 2) return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false); // row_half_mirror
    else if constexpr (STEP == 3) return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false); // row_mirror
    else return __builtin_amdgcn_ds_swizzle(v, 0x401F);                                          // lane ^ 16 in 32
}
template <int STEP>
__device__ __forceinline__ float xl32f(float v) { return __int_as_float(xl32<STEP>(__float_as_int(v))); }

// Sum over the 64 lanes of a wave by an xor butterfly (distances 32, 16, .., 1), the same in every lane.
__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave in lane order, by DPP: Hillis-Steele shifts within each row of 16
// (lanes shifted in from outside the row read 0), then row 0's and row 2's totals added into rows 1 and 3, then
// lane 31's into rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1 and 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2 and 3
    return v;
}

}  // namespace strata
