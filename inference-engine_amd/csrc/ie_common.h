// Device helpers shared by the gfx950 attention kernels: bf16 conversion, DPP lane exchange,
// wave reductions with a fixed order, and host-side argument checking for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ie_attn.h"

#define IE_WAVE 64

namespace ie {

// ---------------------------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16hi(uint32_t packed) {
    return __uint_as_float(packed & 0xffff0000u);
}

typedef __bf16 ie_bf16x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 with round-to-nearest-even: the gfx950 v_cvt_pk_bf16_f32 conversion (one
// instruction per pair, NaN stays NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const ie_bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) { return pack_bf16x2(f, 0.0f) & 0xffffu; }

// ---------------------------------------------------------------------------------------------
// Lane exchange. DPP controls (GFX9): quad_perm = sel0 | sel1<<2 | sel2<<4 | sel3<<6,
// row_mirror = 0x140, row_half_mirror = 0x141, row_ror:n = 0x120 + n.
// ---------------------------------------------------------------------------------------------
enum : int {
    DPP_XOR1 = 0xB1,        // quad_perm [1,0,3,2]
    DPP_XOR2 = 0x4E,        // quad_perm [2,3,0,1]
    DPP_XOR3 = 0x1B,        // quad_perm [3,2,1,0]
    DPP_HALF_MIRROR = 0x141,  // lane i <- lane 7-i within each 8 lanes
    DPP_MIRROR = 0x140,       // lane i <- lane 15-i within each 16 lanes
    DPP_ROR8 = 0x128,         // lane i <- lane (i+8)%16 within each 16 lanes
};

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ float shfl_xor(float x, int m) {
    return __shfl_xor(x, m, IE_WAVE);
}

// gfx950 lane swaps (VALU, no LDS round trip). permlane16_swap(x, x) returns {x of rows 0,0,2,2;
// x of rows 1,1,3,3} (rows of 16 lanes), permlane32_swap(x, x) returns {x of the low half twice;
// x of the high half twice}: combining the pair gives lanes i and i^16 (i^32) the same result.
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__host__ __device__ inline int cdiv_i(int a, int b) { return (a + b - 1) / b; }

// Inclusive prefix sum in lane order, on the VALU: shifts by 1, 2, 4 and 8 lanes inside each
// row of 16 (row_shr; a lane whose source lies outside its row adds 0), then each row's total
// carried into the rows after it with row_bcast:15 (rows 1 and 3) and row_bcast:31 (rows 2
// and 3).
__device__ __forceinline__ int wave_incl_scan_i(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);
    return x;
}

// Sum over each group of 8 consecutive lanes; every lane of the group gets the sum.
__device__ __forceinline__ float sum8(float x) {
    x += dpp<DPP_XOR1>(x);
    x += dpp<DPP_XOR2>(x);
    x += dpp<DPP_HALF_MIRROR>(x);
    return x;
}
// Max over each group of 16 consecutive lanes; every lane of the group gets the max.
__device__ __forceinline__ float max16(float x) {
    x = fmaxf(x, dpp<DPP_XOR1>(x));
    x = fmaxf(x, dpp<DPP_XOR2>(x));
    x = fmaxf(x, dpp<DPP_HALF_MIRROR>(x));
    x = fmaxf(x, dpp<DPP_MIRROR>(x));
    return x;
}
// Integer sum over the wave, every lane gets it (VALU only: the lane swaps for 32 and 16, DPP
// within rows of 16).
__device__ __forceinline__ int wave_sum_i(int x) {
    {
        const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
        x = (int)(r[0] + r[1]);
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)x, false, false);
        x = (int)(r[0] + r[1]);
    }
    x += dppi<DPP_ROR8>(x);
    x += dppi<DPP_HALF_MIRROR>(dppi<DPP_XOR3>(x));
    x += dppi<DPP_XOR2>(x);
    x += dppi<DPP_XOR1>(x);
    return x;
}

// Division by a wave-uniform divisor d >= 1 of numerators 0 <= x < 2^22: the float estimate
// x * (1/d) is within one of floor(x / d), and one compare each way makes it exact.
struct Divisor {
    int d;
    float r;
};
__device__ __forceinline__ Divisor divisor(int d) { return Divisor{d, 1.0f / (float)d}; }
__device__ __forceinline__ int div_floor(int x, const Divisor& D) {
    int q = (int)((float)x * D.r);
    q += (q + 1) * D.d <= x;
    q -= q * D.d > x;
    return q;
}
__device__ __forceinline__ int div_ceil(int x, const Divisor& D) { return div_floor(x + D.d - 1, D); }

// Max over the 64 lanes of the wave (all on the VALU: DPP within rows of 16, then the gfx950
// lane swaps across rows).
__device__ __forceinline__ float wave_max(float x) { return max_xor32(max_xor16(max16(x))); }
// Sum over the 64 lanes in the fixed butterfly order: lane i adds lane i^32, i^16, ..., i^1.
// fp32 addition is commutative, so after each step lanes i and i^m hold the same bits and the
// result is identical in every lane. All on the VALU: the lane swaps for 32 and 16, row_ror:8
// for 8, quad_perm [3,2,1,0] then row_half_mirror (lane i <- 7 - (i ^ 3) = i ^ 4) for 4, and
// quad_perm for 2 and 1.
__device__ __forceinline__ float wave_sum_butterfly(float x) {
    x = sum_xor16(sum_xor32(x));
    x = x + dpp<DPP_ROR8>(x);
    x = x + dpp<DPP_HALF_MIRROR>(dpp<DPP_XOR3>(x));
    x = x + dpp<DPP_XOR2>(x);
    x = x + dpp<DPP_XOR1>(x);
    return x;
}

// ---------------------------------------------------------------------------------------------
// Raw buffer loads: a descriptor over [base, base + bytes); lanes whose offset falls outside the
// range read zeros, which is how the kernels mask rows past a sequence's end without branches.
// ---------------------------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int RSRC_WORD3 = 0x00020000;  // GFX9 buffer descriptor word 3 (32-bit raw data)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, RSRC_WORD3);
}

// ---------------------------------------------------------------------------------------------
// Device-coherent accesses, for partial results that one workgroup writes and another merges in
// the same launch: loads and stores with the device scope bit (sc1), served at the level all
// XCDs share rather than from a possibly stale per-XCD L2 line. The 4- and 8-byte forms are
// agent-scope relaxed atomics; the 16-byte load is a buffer load with that cache policy. The
// writer waits for its stores (wait_stores) before the barrier that precedes its arrival count,
// and the merging workgroup reads only after that count: the order a device-scope release and
// acquire give, without the whole-L2 writeback and invalidate those fences cost.
// ---------------------------------------------------------------------------------------------
constexpr int CPOL_SC1 = 16;  // buffer intrinsic cache policy: device scope
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev64(void* p, uint64_t v) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev64(const void* p) {
    return __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
// Every vector memory access of the wave, stores included, has completed.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Counts the calling workgroup in at `count` (thread 0's device-scope atomic, after a barrier
// that follows every wave's wait_stores) and returns, to every thread, whether it was the last
// of `needed`. The count is a wrapping increment (old >= needed - 1 stores 0), so the last one
// leaves it zero for the next launch in the same operation, and a count left stale by a caller
// (a workspace that was not zeroed) is cleared by the first arrival that meets it instead of
// keeping every later merge from running.
__device__ __forceinline__ bool arrive_last(uint32_t* count, int needed) {
    __shared__ uint32_t s_last;
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __builtin_amdgcn_atomic_inc32(count, (uint32_t)(needed - 1), __ATOMIC_RELAXED,
                                               "agent") == (uint32_t)(needed - 1);
    __syncthreads();
    return s_last != 0;
}

// One entry i = t half + j of the RoPE tables (architecture.py:382-390): the fp32 product of
// position t and inverse frequency j, then cosf / sinf rounded to nearest even bf16 (the
// arithmetic of PyTorch's kernels for angles = positions x inv_freq, cos, sin, cast).
__device__ __forceinline__ void rope_table_entry(const int32_t* __restrict__ pos,
                                                 const float* __restrict__ inv, int64_t i,
                                                 int half, uint16_t* __restrict__ cosv,
                                                 uint16_t* __restrict__ sinv) {
    const int64_t t = i / half;
    const int j = (int)(i - t * half);
    const float a = (float)pos[t] * inv[j];  // a product alone: nothing to contract
    cosv[i] = (uint16_t)f32_to_bf16_rne(cosf(a));
    sinv[i] = (uint16_t)f32_to_bf16_rne(sinf(a));
}

// ---------------------------------------------------------------------------------------------
// Host-side checks.
// ---------------------------------------------------------------------------------------------
void set_error(const char* msg);
hipError_t check_cache(const ie_kv_cache* c);
int device_cu_count();

}  // namespace ie

#define IE_REQUIRE(cond, msg)                      \
    do {                                           \
        if (!(cond)) {                             \
            ::ie::set_error(msg);                  \
            return hipErrorInvalidValue;           \
        }                                          \
    } while (0)
