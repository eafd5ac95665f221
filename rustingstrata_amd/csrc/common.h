// Shared definitions of the strata_hip library: type table, error plumbing, small device helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

namespace strata {

// GGUF type ids (src/quant/mod.rs:15-19) of the types this library decodes.
enum Ty : int { Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, IQ2_XXS = 16, IQ3_S = 21, IQ4_XS = 23 };

// Block elements and bytes (GgmlType::block_elems / block_bytes, src/quant/mod.rs:37-43).
__host__ __device__ constexpr int block_elems(int ty) { return ty == Q8_0 ? 32 : 256; }
__host__ __device__ constexpr int block_bytes(int ty) {
    return ty == Q8_0 ? 34 : ty == Q2_K ? 84 : ty == Q3_K ? 110 : ty == Q4_K ? 144 : ty == Q5_K ? 176
         : ty == Q6_K ? 210 : ty == IQ2_XXS ? 66 : ty == IQ3_S ? 110 : ty == IQ4_XS ? 136 : 0;
}
// Bytes per 256 values: the unit the kernels call a super-block (8 Q8_0 blocks make one, 272 bytes).
__host__ __device__ constexpr int sb_bytes(int ty) { return block_bytes(ty) * (256 / block_elems(ty)); }
inline bool supported(int ty) { return block_bytes(ty) != 0; }
inline uint64_t row_bytes(int ty, uint64_t cols) { return cols / block_elems(ty) * block_bytes(ty); }
const char* type_name(int ty);

// Error state of the C ABI: set_error records the message for strata_last_error and returns -1.
int set_error(const std::string& msg);
int hip_error(hipError_t e, const char* what);
#define STRATA_HIP(call)                                                          \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess) return ::strata::hip_error(e_, #call);              \
    } while (0)

// ---- device helpers ----

__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
    _Float16 h;
    uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}
// Global-memory (address space 1) views of a device address. Loads through them compile to global_load, which
// counts only in vmcnt; loads through a generic pointer become flat_load, which also counts in lgkmcnt, so every
// later LDS wait would stall on them and a prefetch could not overlap LDS work.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(uint64_t addr) {
    return (const __attribute__((address_space(1))) T*)addr;
}
// Read of a value that no kernel of the launch writes, at a wave-uniform address, through the scalar cache
// (s_load: its wait is lgkmcnt, so it does not wait for the wave's vector loads in flight).
template <class T>
__device__ __forceinline__ T sload(const T* p) {
    return *(const __attribute__((address_space(4))) T*)(uintptr_t)p;
}
// LDS (address space 3) view of a generic pointer into shared memory. Keeping LDS reads in their own address space
// stops the compiler from merging them with global reads into flat ones.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(3))) T* lptr(const void* p) {
    return (const __attribute__((address_space(3))) T*)p;
}
// silu(v) = v / (1 + e^-v) with e^-v in double rounded once to f32 (the correctly rounded f32 exp but in vanishingly
// rare cases), for silu(g) * u ahead of a quantization (src/ops.rs:14; swiglu_q src/cuda/kernels.cu:1826-1839).
__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + (float)exp(-(double)v)); }
__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
// Bytes {hi:lo} >> 8 * (sh & 3): the 4 bytes starting at byte sh of the 8-byte pair (v_alignbyte_b32).
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}
// Byte j of the result is 0x01 where bit j of s is set (j < 4).
__device__ __forceinline__ uint32_t bits_to_bytes(uint32_t s) { return ((s & 15u) * 0x00204081u) & 0x01010101u; }
// Bytes of g negated where bit j of s (j < 4) is set. No byte of g is 0, so ~g + 1 per byte never carries.
__device__ __forceinline__ int neg_bytes(uint32_t g, uint32_t s) {
    uint32_t n = bits_to_bytes(s);
    return (int)((g ^ (n * 0xFFu)) + n);
}

// 16 bytes per lane from global address g into LDS at lds + 16 * lane (global_load_lds_dwordx4, LDS base in M0).
// Issued as inline assembly so that the compiler's wait insertion does not tie it to later LDS reads: it would
// otherwise wait for every outstanding load before the first LDS read, and a load issued for a later super-block
// could not overlap this one. The kernel waits for these loads itself (wait_loads) before the barrier that
// publishes them. `lds` must be the same for every lane of the wave.
__device__ __forceinline__ void load_lds16(uint64_t g, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(m0) : "memory", "m0");
}
// The same from a wave-uniform 64-bit base plus a per-lane 32-bit byte offset (the base stays in scalar registers).
__device__ __forceinline__ void load_lds16_so(uint64_t base, uint32_t off, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    // readfirstlane returns int: widen through uint32_t, or bit 31 of the low half would spread into the high half
    const uint64_t sb = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32)) << 32) |
                        (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(sb), "s"(m0) : "memory", "m0");
}
// 4 bytes per lane from a wave-uniform base plus a per-lane offset into LDS at lds + 4 * lane (global_load_lds_dword).
__device__ __forceinline__ void load_lds4_so(uint64_t base, uint32_t off, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    const uint64_t sb = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32)) << 32) |
                        (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" : : "v"(off), "s"(sb), "s"(m0) : "memory", "m0");
}
// Block barrier after this wave's LDS operations complete, without waiting for its loads in flight (a
// __syncthreads() fence would also wait for every outstanding vector memory operation).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }
// This wave's loads into LDS are complete (vmcnt 0; the barrier that follows publishes them to the block).
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// Wait for this wave's LDS reads: before global_load_lds overwrites LDS bytes the wave has just read, since the
// async write can land ahead of a read still queued in the LDS (a barrier carries this wait; a wave-local reuse does not).
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// All but this wave's N most recent vector memory operations are complete (vector loads complete in order).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

}  // namespace strata
