// int8 KV cache writes and reads for gfx950.
//
//   quantize_kv_prefill_kernel   prefill quantize-on-write (+ K calibration on a first chunk)
//   kcal_max_kernel              first-chunk K calibration ahead of the quantize, long steps
//   quantize_kv_stream_kernel    the quantize launch of long steps (resident grid, prefetch)
//   fused_rope_kv_decode_kernel  decode q/k RMSNorm + RoPE, q * calibration, K/V quantize
//   dequantize_kv_prefix_kernel  int8 prefix -> bf16
//
// Bit-level contract: every value written is the one IEEE round-to-nearest-even fp32
// operations in the order stated at each step produce (no contraction into fused multiply-add),
// so it is reproducible on the host; the prefill quantizers reach the IEEE quotients through
// reciprocals where that is exact (div_recip). Each row of 128 channels is handled by 16 lanes x 8 channels
// (prefill) or by one wave, 2 channels per lane (decode).
#include "ie_common.h"
#include "kv_math.h"

namespace ie {

constexpr int HEAD_DIM = 128;
constexpr int QP_THREADS = 256;
constexpr int QP_ROWS = QP_THREADS / 16;   // token rows per pass of a workgroup
constexpr int QP_BLOCK = 32;               // chunk rows per workgroup
constexpr int QP_CAL_BATCH = 32;           // calibration rows in flight per thread
// Steps of at most this many packed tokens compute a first chunk's calibration inside the
// quantize launch (every block re-reads the chunk's K: (len / 32) x len x 256 B per KV head);
// longer steps compute it in two launches of linear cost first.
constexpr int64_t QP_INLINE_CAL_MAX_TOKENS = 1536;
constexpr int QP_CAL_BLOCK = 256;  // chunk rows per workgroup of the separate calibration launch
// The long steps' quantize launch (quantize_kv_stream_kernel): rows per block, and workgroups
// per CU of its resident grid (measured on a 12,288-token step: 32 rows and 4 workgroups per CU
// against 64 rows at 3 or 4 per CU +4-7 %, 128 rows at 2 per CU +22 %, 2 per CU +5 %; workgroups
// that hold every KV head of their tokens, so that a wave reads 1 KB of a token row, +6 %).
#ifndef IE_QS_BLOCK
#define IE_QS_BLOCK 32
#endif
#ifndef IE_QS_WG_PER_CU
#define IE_QS_WG_PER_CU 4
#endif
// The quantizers store int8 rows and scales with the non-temporal cache policy: the cache is
// written once here and read by later steps' attention, not by this launch (12,288-token step
// 22.8 -> 20.4 us; config 4 level). Non-temporal loads of the bf16 rows measured slower.
#ifndef IE_KV_NT_STORE
#define IE_KV_NT_STORE 1
#endif
constexpr int QS_BLOCK = IE_QS_BLOCK;
constexpr int QS_WG_PER_CU = IE_QS_WG_PER_CU;

typedef uint32_t kv_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void row_store8(int8_t* p, uint2 v) {
    if constexpr (IE_KV_NT_STORE)
        __builtin_nontemporal_store(kv_u32x2{v.x, v.y}, reinterpret_cast<kv_u32x2*>(p));
    else
        *reinterpret_cast<uint2*>(p) = v;
}
__device__ __forceinline__ void scale_store(float* p, float v) {
    if constexpr (IE_KV_NT_STORE) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// 8 consecutive bf16 (16 bytes), packed two per word.
struct Row8 {
    uint32_t w[4];
};
__device__ __forceinline__ Row8 load_bf16x8(const uint16_t* p) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    return Row8{{u.x, u.y, u.z, u.w}};
}

__device__ __forceinline__ uint2 pack_i8x8(const int32_t* q) {
    uint2 o;
    o.x = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((uint32_t)q[3] << 24);
    o.y = (q[4] & 0xff) | ((q[5] & 0xff) << 8) | ((q[6] & 0xff) << 16) | ((uint32_t)q[7] << 24);
    return o;
}

// Quantize 8 channels held by this lane of a 16-lane row group; returns the row scale.
__device__ __forceinline__ float quantize_row8(const float* x, int32_t* q) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(x[j]));
    a = max16(a);
    const float s = fmaxf(a, 1e-6f) / 127.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = quant1(x[j], s);
    return s;
}

// x / b from y = 1 / b (IEEE division): q0 = x * y, r = fma(-q0, b, x) (exact), q0 + r * y
// fused (Markstein's correction step). This is the IEEE quotient unless the quotient or the
// remainder underflows or overflows: 3 instructions where an IEEE division compiles to 11. The
// quantizers use it only for rows whose |x| stay below 2^100 (RECIP_MAX_BITS; row_needs_ieee
// sends other rows, inf and NaN included, to the IEEE division), where tests/divcheck checks it
// on the host against the IEEE quotient: every bf16 x against every calibration the writes
// produce (wherever the quotient is at least 2^-64: smaller ones quantize to 0 against any row
// scale, and a row maximum below 1e-6 is raised to 1e-6 before it becomes a scale), the int8
// value of every bf16 x against every bf16 row maximum, and 10^9 random fp32 pairs each for K
// rows after the calibration division and for other calibrations.
__device__ __forceinline__ float div_recip(float x, float b, float y) {
#pragma clang fp contract(off)
    const float q0 = x * y;
    const float r = __builtin_fmaf(-q0, b, x);
    return __builtin_fmaf(r, y, q0);
}
constexpr uint32_t RECIP_MAX_BITS = 0x71800000u;  // fp32 bits of 2^100

// Whether the 16-lane row group of this lane holds a bf16 value (8 per lane, packed in w) the
// reciprocal division does not serve: |x| >= 2^100, inf or NaN. Uniform within the row group.
__device__ __forceinline__ bool row_needs_ieee(const uint32_t (&w)[4]) {
    bool big = false;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        big |= (w[j] & 0x7fff0000u) >= RECIP_MAX_BITS || ((w[j] << 16) & 0x7fffffffu) >= RECIP_MAX_BITS;
    const uint64_t m = __ballot(big);
    return ((m >> (threadIdx.x & 48)) & 0xffffu) != 0;
}

// quantize_row8 through the scale's reciprocal, for the rows row_needs_ieee lets through (also
// after the calibration division): the same int8 values and scale, packed as pack_i8x8 packs
// them. Two exact shortcuts: rint (half to even) of a quotient q with |q| < 2^22 is the sum
// q + 1.5 * 2^23 rounded to nearest even, whose low mantissa byte is the integer as int8 (the
// sum is 0x4B400000 + rint(q) in bits), so a byte permute packs four of them; and the clamp to
// +-127 never binds: s = max(a, 1e-6) / 127 with a = max |x| gives |x / s| <= 127 (1 + 2^-24).
__device__ __forceinline__ float quantize_row8_recip(const float* x, uint2& packed) {
#pragma clang fp contract(off)
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(x[j]));
    a = max16(a);
    const float s = fmaxf(a, 1e-6f) / 127.0f;
    const float y = 1.0f / s;
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = __float_as_uint(div_recip(x[j], s, y) + 12582912.0f);
    // bytes 0 of b0..b3 (and b4..b7): two permutes to pair them, one to join the pairs
    packed.x = __builtin_amdgcn_perm(__builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u),
                                     __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u), 0x05040100u);
    packed.y = __builtin_amdgcn_perm(__builtin_amdgcn_perm(b[7], b[6], 0x0c0c0400u),
                                     __builtin_amdgcn_perm(b[5], b[4], 0x0c0c0400u), 0x05040100u);
    return s;
}

// One row of K and V (8 channels of this lane): K divided by the calibration (cal, its
// reciprocal rcal), both quantized and stored with their scales at column col. The reciprocal
// forms serve the row unless it holds a value they do not (row_needs_ieee).
__device__ __forceinline__ void quantize_store_kv_row(const uint32_t (&kw)[4],
                                                      const uint32_t (&vw)[4], const float* cal,
                                                      const float* rcal, int8_t* kc, int8_t* vc,
                                                      float* ks, float* vs, int64_t col,
                                                      int64_t stride_tok, int c16) {
#pragma clang fp contract(off)
    float xk[8], xv[8];
    int32_t qv[8];
    uint2 packed;
    float sk, sv;
    if (!row_needs_ieee(kw)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xk[2 * j] = div_recip(bf16lo(kw[j]), cal[2 * j], rcal[2 * j]);
            xk[2 * j + 1] = div_recip(bf16hi(kw[j]), cal[2 * j + 1], rcal[2 * j + 1]);
        }
        sk = quantize_row8_recip(xk, packed);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xk[2 * j] = bf16lo(kw[j]) / cal[2 * j];
            xk[2 * j + 1] = bf16hi(kw[j]) / cal[2 * j + 1];
        }
        sk = quantize_row8(xk, qv);
        packed = pack_i8x8(qv);
    }
    row_store8(kc + col * stride_tok, packed);
    if (c16 == 0) scale_store(ks + col, sk);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        xv[2 * j] = bf16lo(vw[j]);
        xv[2 * j + 1] = bf16hi(vw[j]);
    }
    if (!row_needs_ieee(vw)) {
        sv = quantize_row8_recip(xv, packed);
    } else {
        sv = quantize_row8(xv, qv);
        packed = pack_i8x8(qv);
    }
    row_store8(vc + col * stride_tok, packed);
    if (c16 == 0) scale_store(vs + col, sv);
}

// The prefilling entries' chunks are cut into blocks of ROWS rows, numbered entry by entry.
// Block u's entry b (-1 past the last block), its index z within the entry, and the entry's
// chunk start, length, cache slot and cached length. Every wave scans the entries' block counts
// (identical result); the entry fields come from the same independent loads, so the data loads
// that follow are the second round trip to memory.
struct QpBlock {
    int b, z, start, len, slot, c0;
};
template <int ROWS>
__device__ __forceinline__ QpBlock qp_locate(int u, const int32_t* __restrict__ cu_seqlens,
                                             const int32_t* __restrict__ slot_ids,
                                             const int32_t* __restrict__ cached_lens,
                                             const int32_t* __restrict__ num_decoding,
                                             int num_entries) {
    const int lane = threadIdx.x & 63;
    const int nd = __builtin_amdgcn_readfirstlane(num_decoding[0]);
    int b = -1, z = 0, before = 0, start = 0, len = 0, slot = 0, c0 = 0;
    for (int base = 0; base < num_entries && b < 0; base += IE_WAVE) {
        const int e = base + lane;
        int s0 = 0, s1 = 0, sl = 0, cl = 0;
        if (e < num_entries) {
            s0 = cu_seqlens[e];
            s1 = cu_seqlens[e + 1];
            sl = slot_ids[e];
            cl = cached_lens[e];
        }
        const int nb = e >= nd && e < num_entries ? cdiv_i(s1 - s0, ROWS) : 0;
        const int incl = wave_incl_scan_i(nb) + before;
        const unsigned long long hit = __ballot(u < incl && u >= incl - nb);
        if (hit) {
            const int src = __builtin_ctzll(hit);
            auto from = [&](int x) { return __builtin_amdgcn_readlane(x, src); };
            b = from(e);
            z = u - from(incl - nb);
            start = from(s0);
            len = from(s1 - s0);
            slot = from(sl);
            c0 = from(cl);
        }
        before = __builtin_amdgcn_readlane(incl, 63);
    }
    return QpBlock{b, z, start, len, slot, c0};
}

// Calibration rows longer than a few blocks are computed ahead of the quantize launch, in
// linear time: kcal_max_kernel's workgroups (one per block of QP_CAL_BLOCK rows) take the max |k|
// per channel of their rows and combine them in the entry's calibration row with an atomic max
// on the bits of the NEGATED maximum: the bits of negative floats are all above those of
// positive ones and grow with the magnitude, so whatever positive calibration the row held
// before (an earlier sequence's) loses to the first block's value, and the row ends up holding
// -(max over the chunk) (-0 for an all-zero chunk) with no initialization launch. Max is exact
// and order-free, so the result equals the sequential one. The quantize launch reads such a row
// as max(1e-3, -v) (cal_of) and the workgroup holding the chunk's first block stores that,
// positive, back into the row. Blocks of 256 rows keep the atomics per calibration word few
// (they serialize at the memory side).
__device__ __forceinline__ float cal_of(float v) {
    return (__float_as_uint(v) >> 31) ? fmaxf(1e-3f, -v) : v;
}

// grid (Hkv, cdiv(N, QP_CAL_BLOCK) + num_entries), block 256.
__global__ __launch_bounds__(QP_THREADS) void kcal_max_kernel(
    const uint16_t* __restrict__ k, int64_t k_st, int64_t k_sh,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cached_lens, const int32_t* __restrict__ num_decoding,
    int num_entries, ie_kv_cache c) {
    const int h = blockIdx.x;
    const QpBlock q = qp_locate<QP_CAL_BLOCK>(blockIdx.y, cu_seqlens, slot_ids, cached_lens,
                                              num_decoding, num_entries);
    if (q.b < 0 || q.c0 != 0) return;
    const int tid = threadIdx.x, c16 = tid & 15, r = tid >> 4;
    const int t0 = q.z * QP_CAL_BLOCK, t1 = min(q.len, t0 + QP_CAL_BLOCK);
    const uint16_t* kh = k + (int64_t)q.start * k_st + h * k_sh + 8 * c16;
    float mx[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) mx[j] = 0.0f;
    uint4 w[QP_CAL_BLOCK / QP_ROWS];  // all of the thread's rows in flight at once
#pragma unroll
    for (int i = 0; i < QP_CAL_BLOCK / QP_ROWS; ++i) {
        const int t = t0 + r + i * QP_ROWS;
        w[i] = t < t1 ? *reinterpret_cast<const uint4*>(kh + (int64_t)t * k_st)
                      : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < QP_CAL_BLOCK / QP_ROWS; ++i) {
        const uint32_t x[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mx[2 * j] = fmaxf(mx[2 * j], fabsf(bf16lo(x[j])));
            mx[2 * j + 1] = fmaxf(mx[2 * j + 1], fabsf(bf16hi(x[j])));
        }
    }
    __shared__ float s_red[QP_ROWS][HEAD_DIM];
#pragma unroll
    for (int j = 0; j < 8; ++j) s_red[r][8 * c16 + j] = mx[j];
    __syncthreads();
    if (tid < HEAD_DIM) {
        float m = 0.0f;
#pragma unroll
        for (int rr = 0; rr < QP_ROWS; ++rr) m = fmaxf(m, s_red[rr][tid]);
        float* calp = c.k_calibration + q.slot * c.cal_stride_slot + h * c.cal_stride_head;
        atomicMax(reinterpret_cast<unsigned int*>(calp + tid), __float_as_uint(-m));
    }
}

// grid (Hkv, cdiv(N, ROWS) + num_entries), block 256: workgroup (h, u) quantizes block u of ROWS
// rows for kv head h (kernels.py:786-823), or exits when there are fewer blocks. With INLINE_CAL, every
// block of an entry with cached_len == 0 computes the chunk's calibration (kernels.py:764-780)
// itself and block 0 stores it (one launch; each block reads the whole chunk's K, so the host
// takes this form only for short steps); otherwise the calibration row was computed by the two
// launches above and every block reads it.
template <bool INLINE_CAL, int ROWS>
__global__ __launch_bounds__(QP_THREADS) void quantize_kv_prefill_kernel(
    const uint16_t* __restrict__ k, int64_t k_st, int64_t k_sh,
    const uint16_t* __restrict__ v, int64_t v_st, int64_t v_sh,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cached_lens, const int32_t* __restrict__ num_decoding,
    int num_entries, ie_kv_cache c) {
#pragma clang fp contract(off)
    const int h = blockIdx.x;
    const QpBlock q = qp_locate<ROWS>(blockIdx.y, cu_seqlens, slot_ids, cached_lens,
                                      num_decoding, num_entries);
    if (q.b < 0) return;
    const int z = q.z, start = q.start, len = q.len, slot = q.slot, c0 = q.c0;
    const int t0 = z * ROWS;
    const int t1 = min(len, t0 + ROWS);

    const int tid = threadIdx.x;
    const int c16 = tid & 15;  // channels [8*c16, 8*c16+8)
    const int r = tid >> 4;    // row within a pass

    __shared__ float s_red[QP_ROWS][HEAD_DIM];
    __shared__ float s_cal[HEAD_DIM];

    float* calp = c.k_calibration + slot * c.cal_stride_slot + h * c.cal_stride_head;
    const uint16_t* kh = k + (int64_t)start * k_st + h * k_sh + 8 * c16;
    const uint16_t* vh = v + (int64_t)start * v_st + h * v_sh + 8 * c16;

    // this workgroup's rows, two passes at a time: the first pair is loaded before the
    // calibration pass so both sets of loads are in flight together
    Row8 xk[2], xv[2];
    auto load_pair = [&](int t) {
        xk[0] = load_bf16x8(kh + (int64_t)t * k_st);
        xv[0] = load_bf16x8(vh + (int64_t)t * v_st);
        if (t + QP_ROWS < t1) {
            xk[1] = load_bf16x8(kh + (int64_t)(t + QP_ROWS) * k_st);
            xv[1] = load_bf16x8(vh + (int64_t)(t + QP_ROWS) * v_st);
        }
    };
    if (t0 + r < t1) load_pair(t0 + r);

    if (INLINE_CAL && c0 == 0) {
        // max |k| per channel over the whole chunk, QP_CAL_BATCH rows per thread in flight
        float mx[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) mx[j] = 0.0f;
        for (int t = r; t < len; t += QP_ROWS * QP_CAL_BATCH) {
            uint4 u[QP_CAL_BATCH];
#pragma unroll
            for (int i = 0; i < QP_CAL_BATCH; ++i) {
                const int ti = t + i * QP_ROWS;
                u[i] = ti < len ? *reinterpret_cast<const uint4*>(kh + (int64_t)ti * k_st)
                                : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int i = 0; i < QP_CAL_BATCH; ++i) {
                const uint32_t w[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    mx[2 * j] = fmaxf(mx[2 * j], fabsf(bf16lo(w[j])));
                    mx[2 * j + 1] = fmaxf(mx[2 * j + 1], fabsf(bf16hi(w[j])));
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) s_red[r][8 * c16 + j] = mx[j];
        __syncthreads();
        if (tid < HEAD_DIM) {
            float m = 1e-3f;
#pragma unroll
            for (int rr = 0; rr < QP_ROWS; ++rr) m = fmaxf(m, s_red[rr][tid]);
            s_cal[tid] = m;
            if (z == 0) calp[tid] = m;
        }
    } else {
        if (tid < HEAD_DIM) s_cal[tid] = calp[tid];
    }
    __syncthreads();
    float cal[8], rcal[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        cal[j] = s_cal[8 * c16 + j];
        rcal[j] = 1.0f / cal[j];
    }

    int8_t* kc = c.k + slot * c.stride_slot + h * c.stride_head + 8 * c16;
    int8_t* vc = c.v + slot * c.stride_slot + h * c.stride_head + 8 * c16;
    float* ks = c.k_scale + slot * c.scale_stride_slot + h * c.scale_stride_head;
    float* vs = c.v_scale + slot * c.scale_stride_slot + h * c.scale_stride_head;

    for (int t = t0 + r; t < t1; t += 2 * QP_ROWS) {
        const bool two = t + QP_ROWS < t1;
        Row8 ck[2] = {xk[0], xk[1]}, cv[2] = {xv[0], xv[1]};
        if (t + 2 * QP_ROWS < t1) load_pair(t + 2 * QP_ROWS);  // next pair in flight
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            if (p == 1 && !two) break;
            const int64_t col = (int64_t)(c0 + t + p * QP_ROWS);
            quantize_store_kv_row(ck[p].w, cv[p].w, cal, rcal, kc, vc, ks, vs, col, c.stride_tok,
                                  c16);
        }
    }
}

// The streaming form of the quantize launch, for long steps (their first chunks' calibration
// rows come from kcal_max, in the negated form cal_of reads): one resident wave of workgroups, workgroup (h, g) taking
// blocks g, g + G, ... of ROWS rows for kv head h (G = gridDim.y), with the next block's rows and
// calibration in flight while the current block is quantized and stored. Up to 64 entries the
// entry table sits in registers (lane e: entry e), so a block is located without a memory round
// trip; with more entries each block is located by qp_locate. Same arithmetic, in the same
// order, as quantize_kv_prefill_kernel: the same bits.
template <int ROWS>
struct QsRegs {
    uint4 k[ROWS / QP_ROWS], v[ROWS / QP_ROWS];
    float4 cal[2];
};

template <int ROWS>
__global__ __launch_bounds__(QP_THREADS) void quantize_kv_stream_kernel(
    const uint16_t* __restrict__ k, int64_t k_st, int64_t k_sh,
    const uint16_t* __restrict__ v, int64_t v_st, int64_t v_sh,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cached_lens, const int32_t* __restrict__ num_decoding,
    int num_entries, ie_kv_cache c) {
#pragma clang fp contract(off)
    constexpr int RPT = ROWS / QP_ROWS;  // rows per thread and block
    const int h = blockIdx.x, G = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int c16 = tid & 15, r = tid >> 4;

    // the entry table: lane e holds entry e's chunk, slot, cached length and block count
    const bool in_regs = num_entries <= IE_WAVE;  // uniform
    int e_s0 = 0, e_s1 = 0, e_sl = 0, e_cl = 0;
    const int nd = __builtin_amdgcn_readfirstlane(num_decoding[0]);
    if (in_regs && lane < num_entries) {
        e_s0 = cu_seqlens[lane];
        e_s1 = cu_seqlens[lane + 1];
        e_sl = slot_ids[lane];
        e_cl = cached_lens[lane];
    }
    const int e_nb = in_regs && lane >= nd && lane < num_entries ? cdiv_i(e_s1 - e_s0, ROWS) : 0;
    const int e_incl = wave_incl_scan_i(e_nb);
    auto locate = [&](int u) -> QpBlock {
        if (!in_regs)
            return qp_locate<ROWS>(u, cu_seqlens, slot_ids, cached_lens, num_decoding,
                                   num_entries);
        const unsigned long long hit = __ballot(e_nb > 0 && u < e_incl && u >= e_incl - e_nb);
        if (!hit) return QpBlock{-1, 0, 0, 0, 0, 0};
        const int src = __builtin_ctzll(hit);
        auto from = [&](int x) { return __builtin_amdgcn_readlane(x, src); };
        return QpBlock{src, u - from(e_incl - e_nb), from(e_s0), from(e_s1 - e_s0), from(e_sl),
                       from(e_cl)};
    };
    auto load = [&](const QpBlock& q, QsRegs<ROWS>& x) {
        const int t0 = q.z * ROWS, t1 = min(q.len, t0 + ROWS);
        const uint16_t* kh = k + (int64_t)q.start * k_st + h * k_sh + 8 * c16;
        const uint16_t* vh = v + (int64_t)q.start * v_st + h * v_sh + 8 * c16;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int t = t0 + r + i * QP_ROWS;
            if (t < t1) {
                x.k[i] = *reinterpret_cast<const uint4*>(kh + (int64_t)t * k_st);
                x.v[i] = *reinterpret_cast<const uint4*>(vh + (int64_t)t * v_st);
            }
        }
        const float* calp =
            c.k_calibration + q.slot * c.cal_stride_slot + h * c.cal_stride_head + 8 * c16;
        x.cal[0] = *reinterpret_cast<const float4*>(calp);
        x.cal[1] = *reinterpret_cast<const float4*>(calp + 4);
    };
    float rcal[8];
    int rcal_slot = -1;
    auto store = [&](const QpBlock& q, const QsRegs<ROWS>& x) {
        const int t0 = q.z * ROWS, t1 = min(q.len, t0 + ROWS);
        int8_t* kc = c.k + q.slot * c.stride_slot + h * c.stride_head + 8 * c16;
        int8_t* vc = c.v + q.slot * c.stride_slot + h * c.stride_head + 8 * c16;
        float* ks = c.k_scale + q.slot * c.scale_stride_slot + h * c.scale_stride_head;
        float* vs = c.v_scale + q.slot * c.scale_stride_slot + h * c.scale_stride_head;
        // a first chunk's row holds -(max |k|) until its first block's workgroup stores the
        // calibration itself (cal_of reads either form as the same value)
        const float cal[8] = {cal_of(x.cal[0].x), cal_of(x.cal[0].y), cal_of(x.cal[0].z),
                              cal_of(x.cal[0].w), cal_of(x.cal[1].x), cal_of(x.cal[1].y),
                              cal_of(x.cal[1].z), cal_of(x.cal[1].w)};
        if (q.c0 == 0 && q.z == 0) {
            float* calp = c.k_calibration + q.slot * c.cal_stride_slot + h * c.cal_stride_head;
            if (tid < 16)
                *reinterpret_cast<float4*>(calp + 8 * c16) = make_float4(cal[0], cal[1], cal[2], cal[3]);
            else if (tid < 32)
                *reinterpret_cast<float4*>(calp + 8 * c16 + 4) = make_float4(cal[4], cal[5], cal[6], cal[7]);
        }
        if (q.slot != rcal_slot) {  // the calibration's reciprocals, once per entry
#pragma unroll
            for (int j = 0; j < 8; ++j) rcal[j] = 1.0f / cal[j];
            rcal_slot = q.slot;
        }
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int t = t0 + r + i * QP_ROWS;
            if (t >= t1) continue;
            const uint32_t kw[4] = {x.k[i].x, x.k[i].y, x.k[i].z, x.k[i].w};
            const uint32_t vw[4] = {x.v[i].x, x.v[i].y, x.v[i].z, x.v[i].w};
            quantize_store_kv_row(kw, vw, cal, rcal, kc, vc, ks, vs, (int64_t)(q.c0 + t),
                                  c.stride_tok, c16);
        }
    };
    // two register sets alternate: block u + G loads into one while block u, in the other, is
    // quantized
    QsRegs<ROWS> xa, xb;
    int u = blockIdx.y;
    QpBlock qa = locate(u);
    if (qa.b < 0) return;
    load(qa, xa);
    for (;;) {
        const QpBlock qb = locate(u + G);
        if (qb.b >= 0) load(qb, xb);
        store(qa, xa);
        if (qb.b < 0) return;
        u += G;
        qa = locate(u + G);
        if (qa.b >= 0) load(qa, xa);
        store(qb, xb);
        if (qa.b < 0) return;
        u += G;
    }
}

// grid (B, ceil((Hq + Hkv) / 4)), block 256: wave w of workgroup y handles head row
// r = 4y + w; r < Hq is query head r, else kv head r - Hq (its K and V). Lane i holds channels
// i and i + 64 (the two halves RoPE pairs, kernels.py:410-436).
__global__ __launch_bounds__(256) void fused_rope_kv_decode_kernel(
    const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_sh,
    const uint16_t* __restrict__ k, int64_t k_sb, int64_t k_sh,
    const uint16_t* __restrict__ v, int64_t v_sb, int64_t v_sh,
    const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    const uint16_t* __restrict__ cosp, int64_t cos_sb,
    const uint16_t* __restrict__ sinp, int64_t sin_sb,
    const int32_t* __restrict__ slot_ids, const int32_t* __restrict__ cached_lens,
    const int32_t* __restrict__ num_decoding, int hq, int ratio, float eps, ie_kv_cache c,
    uint16_t* __restrict__ out, int64_t o_sb, int64_t o_sh) {
#pragma clang fp contract(off)
    const int b = blockIdx.x;  // < batch: every per-sequence load below is in bounds
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int hkv = (int)c.num_kv_heads;
    if (row >= hq + hkv) return;
    const bool is_q = row < hq;
    const int j = is_q ? row / ratio : row - hq;  // kv head whose calibration applies

    // Every load that does not depend on another is issued before the first wait: the step's
    // count, the sequence's slot and length, and the row data (the calibration row, which
    // needs the slot, is the only second round trip).
    const int nd = num_decoding[0];
    const int slot = slot_ids[b];
    const int64_t col = cached_lens[b];
    const uint16_t* src = is_q ? q + b * q_sb + row * q_sh : k + b * k_sb + j * k_sh;
    const uint16_t* w = is_q ? qw : kw;
    const uint16_t x1 = src[lane], x2 = src[lane + 64], w1 = w[lane], w2 = w[lane + 64];
    const uint16_t cv = cosp[b * cos_sb + lane], sv = sinp[b * sin_sb + lane];
    uint16_t vr1 = 0, vr2 = 0;
    if (!is_q) {
        const uint16_t* vp = v + b * v_sb + j * v_sh;
        vr1 = vp[lane];
        vr2 = vp[lane + 64];
    }
    if (b >= nd) return;
    const float* cal = c.k_calibration + slot * c.cal_stride_slot + j * c.cal_stride_head;
    const float c1 = cal[lane], c2 = cal[lane + 64];
    // RMSNorm (kernels.py:417-419 / :426-428), RoPE with bf16 cos/sin (kernels.py:430-436)
    float o1, o2;
    norm_rope_row(bf16_to_f32(x1), bf16_to_f32(x2), bf16_to_f32(w1), bf16_to_f32(w2),
                  bf16_to_f32(cv), bf16_to_f32(sv), eps, o1, o2);
    if (is_q) {
        // q folded with the channel calibration, stored bf16 (kernels.py:440-447).
        uint16_t* o = out + b * o_sb + row * o_sh;
        o[lane] = (uint16_t)f32_to_bf16_rne(o1 * c1);
        o[lane + 64] = (uint16_t)f32_to_bf16_rne(o2 * c2);
        return;
    }
    // K: rope(norm(k)) / cal -> int8 at column cached_len (kernels.py:449-470).
    const int64_t base = slot * c.stride_slot + j * c.stride_head + col * c.stride_tok;
    const int64_t sidx = slot * c.scale_stride_slot + j * c.scale_stride_head + col;
    {
        int32_t q1, q2;
        const float s = quantize_row_wave(o1 / c1, o2 / c2, q1, q2);
        c.k[base + lane] = (int8_t)q1;
        c.k[base + lane + 64] = (int8_t)q2;
        if (lane == 0) c.k_scale[sidx] = s;
    }
    // V: int8 with its own scale (kernels.py:472-480).
    {
        int32_t q1, q2;
        const float s = quantize_row_wave(bf16_to_f32(vr1), bf16_to_f32(vr2), q1, q2);
        c.v[base + lane] = (int8_t)q1;
        c.v[base + lane + 64] = (int8_t)q2;
        if (lane == 0) c.v_scale[sidx] = s;
    }
}

constexpr int NR_ROWS_PER_WAVE = 8;
constexpr int NR_ROWS_PER_WG = 4 * NR_ROWS_PER_WAVE;

// grid (N, ceil((Hq + Hkv) / 32)), block 256 (kernels.py:547-646): wave w of workgroup (t, y)
// normalizes and rotates head rows r = 32y + w + 4i (i < 8) of packed token t; r < Hq is query
// head r, else key head r - Hq. All of the wave's row loads are issued before the first row is
// computed. Lane i holds channels i and i + 64. Every lane holds every row's sum of squares, so
// lane i computes rstd of row i only (one IEEE sqrt and division per lane instead of one per
// row) and the rows read it back with v_readlane.
__global__ __launch_bounds__(256) void fused_norm_rope_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t q_st, int64_t q_sh,
    const uint16_t* __restrict__ k, int64_t k_st, int64_t k_sh,
    const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    const uint16_t* __restrict__ cosp, int64_t cos_st,
    const uint16_t* __restrict__ sinp, int64_t sin_st, int hq, int hkv, float eps,
    uint16_t* __restrict__ qo, int64_t qo_st, int64_t qo_sh,
    uint16_t* __restrict__ ko, int64_t ko_st, int64_t ko_sh) {
    const int64_t t = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int r0 = NR_ROWS_PER_WG * blockIdx.y + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rows = hq + hkv;
    uint16_t a[NR_ROWS_PER_WAVE], b[NR_ROWS_PER_WAVE];
#pragma unroll
    for (int i = 0; i < NR_ROWS_PER_WAVE; ++i) {
        const int r = r0 + 4 * i;
        if (r < rows) {
            const uint16_t* src = r < hq ? q + t * q_st + r * q_sh : k + t * k_st + (r - hq) * k_sh;
            a[i] = src[lane];
            b[i] = src[lane + 64];
        }
    }
    const float cs = bf16_to_f32(cosp[t * cos_st + lane]);
    const float sn = bf16_to_f32(sinp[t * sin_st + lane]);
    const float qw1 = bf16_to_f32(qw[lane]), qw2 = bf16_to_f32(qw[lane + 64]);
    const float kw1 = bf16_to_f32(kw[lane]), kw2 = bf16_to_f32(kw[lane + 64]);
    float my_ss = 0.f;  // lane i: the sum of squares of row i
#pragma unroll
    for (int i = 0; i < NR_ROWS_PER_WAVE; ++i) {
        const int r = r0 + 4 * i;
        if (r >= rows) break;
        const float ss = row_sumsq(bf16_to_f32(a[i]), bf16_to_f32(b[i]));
        my_ss = lane == i ? ss : my_ss;
    }
    const float my_rstd = row_rstd(my_ss, eps);
#pragma unroll
    for (int i = 0; i < NR_ROWS_PER_WAVE; ++i) {
        const int r = r0 + 4 * i;
        if (r >= rows) break;
        const bool is_q = r < hq;
        const float rstd = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_rstd), i));
        float o1, o2;
        row_norm_rope(bf16_to_f32(a[i]), bf16_to_f32(b[i]), rstd, is_q ? qw1 : kw1,
                      is_q ? qw2 : kw2, cs, sn, o1, o2);
        uint16_t* dst = is_q ? qo + t * qo_st + r * qo_sh : ko + t * ko_st + (r - hq) * ko_sh;
        dst[lane] = (uint16_t)f32_to_bf16_rne(o1);
        dst[lane + 64] = (uint16_t)f32_to_bf16_rne(o2);
    }
}

constexpr int DQ_TOKENS = 64;

// grid (num_entries, Hkv, ceil(max_len / 64)), block 256 (kernels.py:868-932): 16 lanes x 8
// channels per token, 16 tokens per pass.
__global__ __launch_bounds__(256) void dequantize_kv_prefix_kernel(
    ie_kv_cache c, const int32_t* __restrict__ cu_cached, const int32_t* __restrict__ slot_ids,
    uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out, int64_t o_sh, int64_t o_st) {
#pragma clang fp contract(off)
    const int b = blockIdx.x, h = blockIdx.y;
    const int out_start = cu_cached[b];
    const int n = cu_cached[b + 1] - out_start;
    const int tbase = blockIdx.z * DQ_TOKENS;
    if (tbase >= n) return;
    const int slot = slot_ids[b];
    const int c16 = threadIdx.x & 15, r = threadIdx.x >> 4;
    const float* calp = c.k_calibration + slot * c.cal_stride_slot + h * c.cal_stride_head;
    float cal[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cal[j] = calp[8 * c16 + j];
    const int8_t* kc = c.k + slot * c.stride_slot + h * c.stride_head + 8 * c16;
    const int8_t* vc = c.v + slot * c.stride_slot + h * c.stride_head + 8 * c16;
    const float* ks = c.k_scale + slot * c.scale_stride_slot + h * c.scale_stride_head;
    const float* vs = c.v_scale + slot * c.scale_stride_slot + h * c.scale_stride_head;
    for (int t = tbase + r; t < min(n, tbase + DQ_TOKENS); t += 16) {
        const uint2 kq = *reinterpret_cast<const uint2*>(kc + (int64_t)t * c.stride_tok);
        const uint2 vq = *reinterpret_cast<const uint2*>(vc + (int64_t)t * c.stride_tok);
        const float sk = ks[t], sv = vs[t];
        uint32_t ko[4], vo[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const uint32_t kw = j < 4 ? kq.x : kq.y, vw = j < 4 ? vq.x : vq.y;
            const int sh = (j & 3) * 8;
            const float k0 = (float)(int8_t)(kw >> sh), k1 = (float)(int8_t)(kw >> (sh + 8));
            const float v0 = (float)(int8_t)(vw >> sh), v1 = (float)(int8_t)(vw >> (sh + 8));
            ko[j / 2] = pack_bf16x2((k0 * sk) * cal[j], (k1 * sk) * cal[j + 1]);
            vo[j / 2] = pack_bf16x2(v0 * sv, v1 * sv);
        }
        const int64_t o = h * o_sh + (int64_t)(out_start + t) * o_st + 8 * c16;
        *reinterpret_cast<uint4*>(k_out + o) = make_uint4(ko[0], ko[1], ko[2], ko[3]);
        *reinterpret_cast<uint4*>(v_out + o) = make_uint4(vo[0], vo[1], vo[2], vo[3]);
    }
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace ie

using namespace ie;

extern "C" hipError_t ie_quantize_kv_prefill(
    const ie_bf16* k, int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* v,
    int64_t v_stride_tok, int64_t v_stride_head, int64_t num_tokens, const int32_t* cu_seqlens,
    const int32_t* slot_ids, const int32_t* cached_lens, const int32_t* num_decoding,
    int32_t num_entries, const ie_kv_cache* cache, hipStream_t stream) {
    hipError_t e = check_cache(cache);
    if (e != hipSuccess) return e;
    IE_REQUIRE(num_entries >= 0 && num_tokens >= 0, "negative sizes");
    if (num_entries == 0) return hipSuccess;
    IE_REQUIRE(k && v && cu_seqlens && slot_ids && cached_lens && num_decoding, "null pointer");
    IE_REQUIRE(aligned16(k) && aligned16(v) && k_stride_tok % 8 == 0 && k_stride_head % 8 == 0 &&
                   v_stride_tok % 8 == 0 && v_stride_head % 8 == 0,
               "k/v rows must be 16-byte aligned with contiguous head_dim");
    // sum over entries of cdiv(len, 32) <= cdiv(N, 32) + num_entries
    const int64_t blocks = (num_tokens + QP_BLOCK - 1) / QP_BLOCK + num_entries;
    IE_REQUIRE(blocks <= 65535, "too many tokens (at most 65535 blocks of 32 rows per step)");
    // kv head fastest: the workgroups in flight together cover whole 2 KB token rows of k and v
    // (measured 5-6 % faster than block fastest at config 4 and on a 12,288-token step)
    dim3 grid((unsigned)cache->num_kv_heads, (unsigned)std::max<int64_t>(1, blocks));
    if (num_tokens <= QP_INLINE_CAL_MAX_TOKENS) {
        hipLaunchKernelGGL((quantize_kv_prefill_kernel<true, QP_BLOCK>), grid, dim3(QP_THREADS),
                           0, stream,
                           (const uint16_t*)k, k_stride_tok, k_stride_head, (const uint16_t*)v,
                           v_stride_tok, v_stride_head, cu_seqlens, slot_ids, cached_lens,
                           num_decoding, num_entries, *cache);
        return hipGetLastError();
    }
    const int64_t cal_blocks = (num_tokens + QP_CAL_BLOCK - 1) / QP_CAL_BLOCK + num_entries;
    hipLaunchKernelGGL(kcal_max_kernel, dim3(cache->num_kv_heads, (unsigned)cal_blocks),
                       dim3(QP_THREADS), 0, stream, (const uint16_t*)k,
                       k_stride_tok, k_stride_head, cu_seqlens, slot_ids, cached_lens,
                       num_decoding, num_entries, *cache);
    // the streaming form: one resident wave of workgroups looping over blocks
    const int hkv = (int)cache->num_kv_heads;
    const int64_t sblocks = (num_tokens + QS_BLOCK - 1) / QS_BLOCK + num_entries;
    const int64_t resident =
        std::max<int64_t>(1, (int64_t)device_cu_count() * QS_WG_PER_CU / hkv);
    const dim3 sgrid((unsigned)hkv, (unsigned)std::min(sblocks, resident));
    hipLaunchKernelGGL((quantize_kv_stream_kernel<QS_BLOCK>), sgrid, dim3(QP_THREADS), 0, stream,
                       (const uint16_t*)k, k_stride_tok, k_stride_head, (const uint16_t*)v,
                       v_stride_tok, v_stride_head, cu_seqlens, slot_ids, cached_lens,
                       num_decoding, num_entries, *cache);
    return hipGetLastError();
}

extern "C" hipError_t ie_fused_rope_kv_decode(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, const ie_bf16* k,
    int64_t k_stride_b, int64_t k_stride_h, const ie_bf16* v, int64_t v_stride_b,
    int64_t v_stride_h, const ie_bf16* q_norm_weight, const ie_bf16* k_norm_weight,
    const ie_bf16* cos, int64_t cos_stride_b, const ie_bf16* sin, int64_t sin_stride_b,
    const int32_t* slot_ids, const int32_t* cached_lens, const int32_t* num_decoding,
    int32_t batch, int32_t num_q_heads, float eps, const ie_kv_cache* cache, ie_bf16* q_out,
    int64_t q_out_stride_b, int64_t q_out_stride_h, hipStream_t stream) {
    hipError_t e = check_cache(cache);
    if (e != hipSuccess) return e;
    IE_REQUIRE(batch >= 0, "negative batch");
    if (batch == 0) return hipSuccess;
    IE_REQUIRE(q && k && v && q_norm_weight && k_norm_weight && cos && sin && slot_ids &&
                   cached_lens && num_decoding && q_out,
               "null pointer");
    IE_REQUIRE(num_q_heads > 0 && num_q_heads % cache->num_kv_heads == 0,
               "num_q_heads must be a multiple of num_kv_heads");
    const int rows = num_q_heads + (int)cache->num_kv_heads;
    dim3 grid(batch, (rows + 3) / 4);
    hipLaunchKernelGGL(fused_rope_kv_decode_kernel, grid, dim3(256), 0, stream,
                       (const uint16_t*)q, q_stride_b, q_stride_h, (const uint16_t*)k,
                       k_stride_b, k_stride_h, (const uint16_t*)v, v_stride_b, v_stride_h,
                       (const uint16_t*)q_norm_weight, (const uint16_t*)k_norm_weight,
                       (const uint16_t*)cos, cos_stride_b, (const uint16_t*)sin, sin_stride_b,
                       slot_ids, cached_lens, num_decoding, num_q_heads,
                       num_q_heads / (int)cache->num_kv_heads, eps, *cache, (uint16_t*)q_out,
                       q_out_stride_b, q_out_stride_h);
    return hipGetLastError();
}

extern "C" hipError_t ie_fused_norm_rope_prefill(
    const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head, const ie_bf16* k,
    int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* q_norm_weight,
    const ie_bf16* k_norm_weight, const ie_bf16* cos, int64_t cos_stride_tok, const ie_bf16* sin,
    int64_t sin_stride_tok, int64_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, float eps, ie_bf16* q_out, int64_t q_out_stride_tok,
    int64_t q_out_stride_head, ie_bf16* k_out, int64_t k_out_stride_tok,
    int64_t k_out_stride_head, hipStream_t stream) {
    IE_REQUIRE(num_tokens >= 0 && num_q_heads >= 0 && num_kv_heads >= 0, "negative sizes");
    IE_REQUIRE(head_dim == 128, "head_dim must be 128");
    if (num_tokens == 0 || num_q_heads + num_kv_heads == 0) return hipSuccess;
    IE_REQUIRE(q && k && q_norm_weight && k_norm_weight && cos && sin && q_out && k_out,
               "null pointer");
    IE_REQUIRE(num_tokens < (1LL << 31), "too many tokens");
    const int rows = num_q_heads + num_kv_heads;
    dim3 grid((unsigned)num_tokens, (unsigned)((rows + NR_ROWS_PER_WG - 1) / NR_ROWS_PER_WG));
    hipLaunchKernelGGL(fused_norm_rope_prefill_kernel, grid, dim3(256), 0, stream,
                       (const uint16_t*)q, q_stride_tok, q_stride_head, (const uint16_t*)k,
                       k_stride_tok, k_stride_head, (const uint16_t*)q_norm_weight,
                       (const uint16_t*)k_norm_weight, (const uint16_t*)cos, cos_stride_tok,
                       (const uint16_t*)sin, sin_stride_tok, num_q_heads, num_kv_heads, eps,
                       (uint16_t*)q_out, q_out_stride_tok, q_out_stride_head, (uint16_t*)k_out,
                       k_out_stride_tok, k_out_stride_head);
    return hipGetLastError();
}

extern "C" hipError_t ie_dequantize_kv_prefix(const ie_kv_cache* cache, const int32_t* cu_cached,
                                              const int32_t* slot_ids, int32_t num_entries,
                                              ie_bf16* k_out, ie_bf16* v_out,
                                              int64_t out_stride_head, int64_t out_stride_tok,
                                              hipStream_t stream) {
    hipError_t e = check_cache(cache);
    if (e != hipSuccess) return e;
    IE_REQUIRE(num_entries >= 0, "negative sizes");
    if (num_entries == 0) return hipSuccess;
    IE_REQUIRE(cu_cached && slot_ids && k_out && v_out, "null pointer");
    IE_REQUIRE(aligned16(k_out) && aligned16(v_out) && out_stride_head % 8 == 0 &&
                   out_stride_tok % 8 == 0,
               "prefix rows must be 16-byte aligned with contiguous head_dim");
    dim3 grid(num_entries, (unsigned)cache->num_kv_heads,
              (unsigned)((cache->max_len + DQ_TOKENS - 1) / DQ_TOKENS));
    hipLaunchKernelGGL(dequantize_kv_prefix_kernel, grid, dim3(256), 0, stream, *cache, cu_cached,
                       slot_ids, (uint16_t*)k_out, (uint16_t*)v_out, out_stride_head,
                       out_stride_tok);
    return hipGetLastError();
}
