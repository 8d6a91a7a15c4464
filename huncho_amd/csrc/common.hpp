// common.hpp - shared device/host helpers for the gfx950 kernels of libhuncho_rocm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace hk {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Accumulator layout of v_mfma_f32_32x32x{16 bf16, 2 f32} (checked on gfx950): lane l
// holds column l % 32 and, in element j, row (j / 4) * 8 + (l / 32) * 4 + j % 4.
__device__ __forceinline__ int acc_row(int j, int g) { return (j >> 2) * 8 + g * 4 + (j & 3); }

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float to_f(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f(f16 x) { return (float)x; }
__device__ __forceinline__ float to_f(float x) { return x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ f16 from_f<f16>(float x) { return (f16)x; }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// a.x b.x + a.y b.y + c with fp32 accumulation (v_dot2_f32_bf16 / v_dot2_f32_f16); the
// products of two 16-bit values are exact in fp32
__device__ __forceinline__ float dot2(bf16x2 a, bf16x2 b, float c) { return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false); }
__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// 32x32x16 MFMA for the two 16-bit operand types (same lane layout).
template <typename T> struct Mma16;
template <> struct Mma16<bf16> {
    typedef bf16x8 v8;
    typedef bf16x4 v4;
    typedef bf16x2 v2;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mma16<f16> {
    typedef f16x8 v8;
    typedef f16x4 v4;
    typedef f16x2 v2;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, output lane 4a + c receives in
// element e the 16-bit element c of the 8 bytes addressed by source lane a + 4e (checked on
// gfx950). Reading rows of a row-major [key][dim] tile this way hands each lane 4 keys of
// one dim: the V^T operand of P.V without a transposed copy.
__device__ __forceinline__ i16x4 lds_read_tr16(const void* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p);
}

// Device fault bits shared with the C ABI (HK_FAULT_*).
constexpr int FAULT_SEQLENS = 1, FAULT_PAGE = 2, FAULT_ROPE = 4, FAULT_TOKEN = 8, FAULT_RANGE = 16;

// Kernel dtype codes shared with the C ABI.
enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// v_rcp_f32 / v_rsq_f32 (about 1 ulp in fp32) instead of the IEEE division sequence; used
// where the result is rounded to a 16-bit activation right after.
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_rsqrt(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ float fast_sigmoid(float x) { return fast_rcp(1.0f + __expf(-x)); }
__device__ __forceinline__ float fast_silu(float x) { return x * fast_rcp(1.0f + __expf(-x)); }

// Sum over each aligned group of 16 lanes, left in every lane of the group: DPP quad_perm
// [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror (every lane adds the same partial
// sums in the same pairing, so the 16 results are identical).
template <int CTRL> __device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum16(float x) {
    x += dpp_mov<0xB1>(x);
    x += dpp_mov<0x4E>(x);
    x += dpp_mov<0x141>(x);
    x += dpp_mov<0x140>(x);
    return x;
}

__device__ __forceinline__ float wave_max32(float v) {
    // combine the two 32-lane halves (lane l and l ^ 32)
    return fmaxf(v, __shfl_xor(v, 32));
}

constexpr int VMCNT0 = 0x0F70;  // s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima)

// One global_load_lds_dwordx4: lane l copies the 16 bytes at g to LDS byte address lds + 16 l
// (lds wave-uniform, in M0). Issued from inline assembly so that the compiler does not make
// every later LDS access wait for the copy; a kernel that uses it waits for its copies
// explicitly (s_waitcnt vmcnt) before the barrier that publishes them. The LDS address is an
// M0 operand ("{m0}"), so the compiler sets M0 itself and knows the asm reads it.
__device__ __forceinline__ void copy_x4(const void* g, unsigned lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
// LDS byte address of a pointer into shared memory
__device__ __forceinline__ unsigned lds_address(const void* p) {
    return (unsigned)(size_t)(const __attribute__((address_space(3))) void*)p;
}

}  // namespace hk

// Status codes shared with include/huncho_rocm.h.
#define HK_OK 0
#define HK_ERR_INVALID 1
#define HK_ERR_UNSUPPORTED 2
#define HK_ERR_DEVICE 3
#define HK_ERR_NOMEM 4
