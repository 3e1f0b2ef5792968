// y[M, N] = x[M, K] . W[N, K]^T for few rows (decode, M <= 64), bf16 in, fp32 accumulation, bf16 out
// (gfx950). Replaces qwen3-1.7b/kernels.py:1373-1443 `skinny_matmul` (the `linear` of
// kernels.py:1451-1458 picks it or the library per shape).
//
// At decode row counts the weight read is the whole cost (one byte of W feeds 2M flops), so the
// kernel streams every weight byte once from HBM and keeps x, which every workgroup needs, in the
// caches. Workgroup n-tile t (grid N / (16 NT), 512 threads) owns W rows [16 NT t, +16 NT); its
// eight waves split K into eight contiguous slices. Per 32-wide k step a wave issues
// v_mfma_f32_16x16x32_bf16 with A = 16 W rows x 32 k (lane (r, g): row r, k 8g..8g+7) and
// B = x^T, 32 k x 16 rows of x per m-tile (the same lane mapping over x's rows), so
// D = y^T (16 n x 16 m).
//
// Loads do not use that lane mapping: a wave load in it touches 16 rows x 64 bytes, and such
// loads moved 15 bytes per clock per CU on this part against 44 for 8 rows x 128 bytes and 50
// for 1 KB contiguous (measured, L2-resident data). So each wave loads a batch of 64 k as
// 8-row x 128-byte pieces (lane (row L / 8, 16-byte chunk L % 8)), stores them in its own LDS
// region (rows of 160 bytes: both the row-wise stores and the fragment reads are free of bank
// conflicts) and reads the MFMA fragments back. Batch b + 1 is loaded into registers while
// batch b goes through LDS and the MFMAs. The eight partial D tiles are summed through LDS in
// wave order and written as bf16. Launch modes below: 8-row n-tiles for narrow weights, the
// gate/up projection with the SiLU-gated product fused (ie_skinny_gemm_silu_mul), and the
// residual add and RMSNorm of a decoder layer fused in (ie_skinny_gemm_fused): an RMSNorm
// before the GEMM costs nothing but a sum of squares over the x fragments the waves already
// hold, once its weight is folded into the GEMM's weight columns, and a residual add after it
// is local to each output element. Weights reordered once into the MFMA fragment order skip the
// LDS round trip (SWZ; the gate/up weight with gate and up rows paired per tile), as does an
// activation written in that order by the gate/up launch for the down projection (YFRAG /
// XFRAG); the LM head loops one workgroup per CU over its row blocks with x in registers
// (LOOP, XREG) and can pick the greedy next token in the same launch (AMAX).
#include "ie_common.h"

namespace ie {

typedef __bf16 sg_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 sg_bf16x2 __attribute__((ext_vector_type(2)));
typedef float sg_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t sg_u32x4 __attribute__((ext_vector_type(4)));

constexpr int SG_WAVES = 8;
constexpr int SG_THREADS = SG_WAVES * IE_WAVE;
constexpr int SG_BK = 64;      // k per batch: 128 bytes of a row, one 8-lane load group
constexpr int SG_LROW = 160;   // LDS row stride (bytes)
constexpr int SG_MAX_TILES = 6;  // weight + x tiles, at most (LDS: 8 waves x 16 tiles' rows x 160 B)
// Weight loads carry the non-temporal cache policy (aux bit 1, "nt"): each weight byte is read
// once per launch, and streaming it past the caches took the LM head from 117 to 105 us and each
// layer projection 0.2-0.9 us lower at 32 rows (x keeps the default policy: every workgroup
// reads it).
#ifndef IE_SKINNY_W_AUX
#define IE_SKINNY_W_AUX 2
#endif

// Launch modes (bits): plain n-tiles of 16 rows; one n-tile of 8 rows (HALF); GLU, the gate/up
// projection with the SiLU-gated product fused: n-tile t pairs gate rows [16 NT t, +16 NT) with
// the up rows nh further (the weight is [gate; up], 2 nh rows) and the workgroup writes
// bf16(silu(g) * u) from the bf16-rounded g and u, as silu_mul does with the GEMM's output;
// NORM, x is a residual stream h whose RMSNorm feeds the GEMM: every fp32 sum of row m is scaled
// by rstd_m = 1 / sqrt(sum_k h[m,k]^2 / K + eps) before it is rounded, the norm's weight having
// been folded into the weight's columns by the caller (y = rstd_m * sum_k h[m,k] (g_k W[n,k]) is
// the GEMM of the normalized rows); RES, y holds the residual stream on entry and each output
// becomes bf16(y + bf16(sum)), in place (add_rms_norm's new residual, kernels.py:1240-1242);
// SWZ, the weight comes in the fragment order skinny_weight_swizzle_kernel writes for NT: 1 KB
// blocks, one per (16-row group, 32-column step), lane (r, g)'s 16 bytes at 16 (16 g + r), the
// NT groups of each workgroup's 16 NT rows interleaved step by step; a wave reads a weight
// fragment as one contiguous 1 KB load, straight into its registers (no LDS round trip for the
// weight; the same fragments, so the same sums, as the row-major form), a workgroup reads only
// its own contiguous rows, and its NT tiles of one step are neighbours in memory; with GLU, the
// gate/up weight in the paired order of skinny_weight_swizzle_kernel (16-row tile T = gate rows
// [8 T, +8) then the matching up rows): each MFMA tile yields 8 gate and their 8 up sums, the
// product needs one lane exchange instead of a second reduction round, and a workgroup writes
// 8 NT output columns (NT = 3 gives Qwen3-1.7B's 6144 columns one workgroup per CU);
// LOOP, the grid is one workgroup per CU and each loops over the row blocks b, b + grid, ...,
// the next block's first batch in flight during the current block's reduction (for weights of
// many more blocks than CUs: the LM head), each block summed exactly as its own workgroup would;
// XREG (with LOOP and SWZ, K = 2048): each wave keeps one K slice for every block and holds its
// x fragments over that slice in registers, loaded once per launch, so the loop streams only
// the weight (no x reloads, no LDS round trip), and NORM's sums of squares are taken once; the
// partial tiles and sums of squares are summed in the slice order of the one-block-per-workgroup
// form, so every block's result bits stay the same.
// XFRAG: x comes in MFMA fragment order (1 KB block per (32-column step S, m-tile mt) at
// block index S * MT + mt, lane (r, g)'s 16 bytes at 16 (16 g + r): row 16 mt + r, columns
// 32 S + 8 g .. + 8), loaded straight into registers like a swizzled weight; YFRAG (paired
// gate/up form): y is written in that order, for a next GEMM that takes it as XFRAG (the MLP's
// down projection), rows past M not written.
// AMAX (with LOOP and XREG: the LM head): also the greedy token of every row, the first column
// of the largest bf16 output (sample's greedy rule at tau = 0: larger value, then smaller index;
// NaN never chosen): each lane keeps its best over its blocks, each workgroup folds its lanes'
// and counts itself into a device-scope 64-bit max per row, and the last workgroup to finish
// writes the tokens, clears the maxima and advances the sampler's seed.
enum : int { SG_PLAIN = 0, SG_HALF = 1, SG_GLU = 2, SG_NORM = 4, SG_RES = 8, SG_SWZ = 16,
             SG_LOOP = 32, SG_XREG = 64, SG_XFRAG = 128, SG_YFRAG = 256, SG_AMAX = 512 };

// AMAX's outputs: per-row maxima keys[M] and a count (zero on entry, left zero), tokens (int64,
// stride os) and the sampler's seed.
struct SgAmax {
    uint64_t* keys;
    uint32_t* count;
    int64_t* out;
    int64_t os;
    int64_t* seed;
};

// (value, index) ordered as the reference's greedy argmax: the larger value, then the smaller
// index; NaN is never larger.
__device__ __forceinline__ bool amax_better(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}
// The pair as a key whose unsigned order is that order: the value's bits made monotonic (-0
// as +0) above the inverted index.
__device__ __forceinline__ uint64_t amax_key(float v, int i) {
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t o = (u >> 31) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
}
constexpr int SG_XREG_K = SG_WAVES * 4 * SG_BK;  // the one K of the XREG form: 4 batches a wave

template <int TT, int MT, int PT>
struct SgLds {
    union {
        uint8_t t[SG_WAVES][16 * TT * SG_LROW];          // per-wave transpose regions
        sg_f32x4 acc[SG_WAVES][PT * MT][IE_WAVE];       // partial D tiles (after the loop)
    };
    float ss[SG_WAVES][16 * MT];  // NORM: each wave's sums of squares of x rows over its K slice
};

// MT m-tiles of 16 rows (M <= 16 MT), NT n-tiles of 16 weight rows per workgroup (every x
// fragment feeds NT MFMAs), or with HALF one n-tile of 8 rows (NT = 1: twice the workgroups for
// narrow weights; the MFMA's other 8 rows compute outputs that are not stored). K a multiple of
// 8 * 32 = 256 (each wave's slice is a multiple of 32).
template <int MT, int NT, int MODE>
__global__ __launch_bounds__(SG_THREADS) void skinny_gemm_kernel(
    const uint16_t* __restrict__ x, int64_t xs, int M, const uint16_t* __restrict__ w, int64_t ws,
    int K, uint16_t* __restrict__ y, int64_t ys, int nh, float eps, int nblk, SgAmax am) {
    constexpr bool HALF = MODE & SG_HALF, GLU = MODE & SG_GLU, NORM = MODE & SG_NORM,
                   RES = MODE & SG_RES, SWZ = MODE & SG_SWZ, LOOP = MODE & SG_LOOP,
                   XREG = MODE & SG_XREG, XFRAG = MODE & SG_XFRAG, YFRAG = MODE & SG_YFRAG,
                   AMAX = MODE & SG_AMAX;
    constexpr bool PAIR = GLU && SWZ;  // gate and up rows paired inside each 16-row tile
    constexpr int WT = GLU && !PAIR ? 2 * NT : NT;  // weight tiles (GLU: NT gate, then NT up)
    static_assert(WT + MT <= SG_MAX_TILES, "LDS transpose region too large");
    static_assert(!HALF || NT == 1, "8-row n-tiles come one per workgroup");
    static_assert(!GLU || SWZ || NT * MT <= SG_WAVES, "GLU: at most one output tile per wave");
    static_assert(!(SWZ && HALF), "the fragment-ordered weight comes in 16-row groups");
    static_assert(!LOOP || !(GLU || RES || HALF || (NORM && !XREG)),
                  "the looping grid: plain launches (NORM: with x in registers)");
    static_assert(!XREG || (LOOP && SWZ), "x in registers: the looping grid over a swizzled weight");
    static_assert(!XFRAG || !(XREG || LOOP), "x in fragment order: one block per workgroup");
    static_assert(!YFRAG || PAIR, "y in fragment order: the paired gate/up form");
    static_assert(!AMAX || (XREG && !GLU && NT * MT <= SG_WAVES),
                  "greedy tokens: the looping LM head, one output tile per wave");
    float abv = -INFINITY;  // AMAX: this lane's best output so far, and its column
    int abi = 0x7fffffff;
    constexpr int XNB = XREG ? SG_XREG_K / SG_WAVES / SG_BK : 1;  // batches of x held per wave
    constexpr int WROWS = HALF ? 8 : 16 * NT;  // weight rows per workgroup (per half in GLU)
    constexpr int TILES = WT + MT;  // W tiles 0..WT-1, then x tiles
    constexpr int T0 = SWZ ? WT : 0;  // the first tile that goes through LDS (its LDS row: 16 (i - T0))
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int lr = lane >> 3, lc = lane & 7;  // load mapping: row lr of 8, 16-byte chunk lc
    const int kw = K / SG_WAVES;
    const rsrc_t rx = make_rsrc(x, (uint32_t)(XFRAG ? K / 32 * MT * 1024 : M * xs * 2));
    int kstep0 = 0;  // XFRAG: the wave's first 32-column step
    rsrc_t rw, ru;
    int loff[TILES][2];
    // Row block bk: W rows [bk WROWS, +WROWS) (GLU: and the up rows nh further) and x rows
    // [0, M): the buffer ranges zero the rows of x past M (SWZ: the same rows, as the
    // workgroup's band). Wave w takes K slice (w + bk) mod 8: neighbouring workgroups read
    // different parts of x at any moment instead of all hitting the same L2 lines (XREG: slice
    // w for every block). loff: byte offsets of this lane's two 8-row halves of every tile at
    // the slice start (SWZ weight tiles: of its two 32-column steps' blocks).
    auto setup = [&](int bk) {
        const int n0 = bk * WROWS,
                  k_begin = (int)(XREG ? wave : (wave + bk) % SG_WAVES) * kw;
        kstep0 = k_begin / 32;
        rw = make_rsrc(w + (int64_t)n0 * ws, (uint32_t)(WROWS * ws * 2));
        ru = make_rsrc(w + ((int64_t)nh + n0) * ws, (uint32_t)(GLU && !PAIR ? WROWS * ws * 2 : 0));
#pragma unroll
        for (int i = 0; i < TILES; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (SWZ && i < WT) {  // group i % NT of the band, step k_begin / 32 + h
                    loff[i][h] = ((k_begin / 32 + h) * NT + i % NT) * 1024 + 16 * lane;
                    continue;
                }
                const int row = 16 * (i < WT ? i % NT : i - WT) + 8 * h + lr;
                loff[i][h] = (row * (int)(i < WT ? ws : xs) + k_begin + 8 * lc) * 2;
            }
    };
    int blk = blockIdx.x;
    setup(blk);
    __shared__ __attribute__((aligned(16))) SgLds<TILES - T0, MT, NT> lds;
    // XREG: the MFMA B fragments of x over the wave's slice, xf[b][t][mt] = x row 16 mt + l16,
    // k = 64 b + 32 t + 8 g .. + 8 of the slice (rows past M read zeros)
    typedef sg_bf16x8 XFrag[2][MT];
    XFrag xf[XNB];
    if constexpr (XREG) {
#pragma unroll
        for (int b = 0; b < XNB; ++b)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    xf[b][t][mt] = __builtin_bit_cast(
                        sg_bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                       rx,
                                       ((16 * mt + l16) * (int)xs + wave * kw + SG_BK * b +
                                        32 * t + 8 * g) * 2,
                                       0, 0));
        if constexpr (NORM) {  // the slice's sums of squares, in the order compute() takes them
            float sq[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) sq[mt] = 0.f;
#pragma unroll
            for (int b = 0; b < XNB; ++b)
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int j = 0; j < 8; j += 2) {
                            const sg_bf16x2 p = {xf[b][t][mt][j], xf[b][t][mt][j + 1]};
                            sq[mt] = __builtin_amdgcn_fdot2_f32_bf16(p, p, sq[mt], false);
                        }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                sq[mt] += __shfl_xor(sq[mt], 16);
                sq[mt] += __shfl_xor(sq[mt], 32);
                if (g == 0) lds.ss[wave][16 * mt + l16] = sq[mt];
            }
        }
    }

    uint8_t* reg = lds.t[wave];
    uint8_t* wdst = reg + lr * SG_LROW + 16 * lc;          // + (16 i + 8 h) rows
    const uint8_t* rsrc = reg + l16 * SG_LROW + 16 * g;   // + 16 i rows + 64 t

    sg_f32x4 acc[WT][MT];
    // NORM: lane (l16, g) sums the squares of the x elements it holds (row 16 mt + l16, 8 of every
    // 32 k of the slice); the four g lanes and eight waves together cover each row once
    float ss[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) ss[mt] = 0.f;

    typedef sg_u32x4 Batch[TILES][2];
    // batch b: k [64 b, 64 b + 64) of the slice; chunks past the slice (or past the last batch)
    // load out of range, i.e. zeros without a memory access
    auto load = [&](Batch& r, int b, bool on = true) {  // on = false: zeros, no memory access
        const bool in = on && SG_BK * b + 8 * lc < kw;
#pragma unroll
        for (int i = 0; i < (XREG ? WT : TILES); ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (HALF && i < NT && h == 1) continue;
                if (SWZ && i < WT) {  // 32-column step h of the batch: one 1 KB block
                    r[i][h] = __builtin_amdgcn_raw_buffer_load_b128(
                        i < NT ? rw : ru,
                        on && SG_BK * b + 32 * h < kw ? loff[i][h] + 2048 * NT * b : -1, 0,
                        IE_SKINNY_W_AUX);
                    continue;
                }
                if (i < WT)
                    r[i][h] = __builtin_amdgcn_raw_buffer_load_b128(
                        i < NT ? rw : ru, in ? loff[i][h] + 128 * b : -1, 0, IE_SKINNY_W_AUX);
                else if (XFRAG)  // 32-column step h of the batch, m-tile i - WT: one 1 KB block
                    r[i][h] = __builtin_amdgcn_raw_buffer_load_b128(
                        rx,
                        on && SG_BK * b + 32 * h < kw
                            ? ((kstep0 + 2 * b + h) * MT + (i - WT)) * 1024 + 16 * lane
                            : -1,
                        0, 0);
                else
                    r[i][h] = __builtin_amdgcn_raw_buffer_load_b128(
                        rx, in ? loff[i][h] + 128 * b : -1, 0, 0);
            }
    };
    auto compute = [&](const Batch& r, const XFrag& xb) {
#pragma unroll
        for (int i = T0; i < (XREG ? T0 : XFRAG ? WT : TILES); ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (HALF && i < NT && h == 1) continue;  // weight rows 8..15: not stored
                *reinterpret_cast<sg_u32x4*>(wdst + (16 * (i - T0) + 8 * h) * SG_LROW) = r[i][h];
            }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            sg_bf16x8 f[TILES];
#pragma unroll
            for (int i = 0; i < TILES; ++i)
                f[i] = i < T0 || (XFRAG && i >= WT) ? __builtin_bit_cast(sg_bf16x8, r[i][t])
                       : XREG ? xb[t][i - T0]
                              : __builtin_bit_cast(sg_bf16x8,
                                                   *reinterpret_cast<const sg_u32x4*>(
                                                       rsrc + 16 * (i - T0) * SG_LROW + 64 * t));
#pragma unroll
            for (int nt = 0; nt < WT; ++nt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f[nt], f[WT + mt],
                                                                         acc[nt][mt], 0, 0, 0);
            if (NORM && !XREG) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const sg_bf16x8 v = f[WT + mt];
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        const sg_bf16x2 p = {v[j], v[j + 1]};
                        ss[mt] = __builtin_amdgcn_fdot2_f32_bf16(p, p, ss[mt], false);
                    }
                }
            }
        }
    };
    // The batch loads are unconditional and each is pinned ahead of the work it overlaps with a
    // sched_barrier: loads under a branch make the compiler's wait counts assume the worst at the
    // join, and left alone the scheduler sinks them below the MFMAs.
    const int nb = (kw + SG_BK - 1) / SG_BK;
    Batch ra, rb, rc, rd;  // rc, rd: XREG only
    load(ra, 0);
    if constexpr (XREG) {  // a ring of four batches, three in flight ahead of the MFMAs
        load(rb, 1);
        load(rc, 2);
    }
    for (;;) {  // once, or (LOOP) over the workgroup's row blocks
#pragma unroll
    for (int nt = 0; nt < WT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = sg_f32x4{0.f, 0.f, 0.f, 0.f};
    const int n0 = blk * WROWS;
    const int next = blk + (int)gridDim.x;
    if constexpr (XREG) {  // nb == XNB == 4; the next block's batches follow this block's
        static_assert(XNB == 4, "the ring holds one block's four batches");
        const bool more = next < nblk;
        load(rd, 3);
        __builtin_amdgcn_sched_barrier(0);
        compute(ra, xf[0]);
        setup(more ? next : blk);
        load(ra, 0, more);
        __builtin_amdgcn_sched_barrier(0);
        compute(rb, xf[1]);
        load(rb, 1, more);
        __builtin_amdgcn_sched_barrier(0);
        compute(rc, xf[2]);
        load(rc, 2, more);
        __builtin_amdgcn_sched_barrier(0);
        compute(rd, xf[3]);
    } else {
        for (int b = 0; b < nb; b += 2) {
            load(rb, b + 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(ra, xf[0]);
            load(ra, b + 2);
            __builtin_amdgcn_sched_barrier(0);
            compute(rb, xf[0]);
        }
    }
    if (LOOP && !XREG && next < nblk) {  // the next block's first batch, in flight during the reduction
        setup(next);
        load(ra, 0);
        __builtin_amdgcn_sched_barrier(0);
    }

    // D lane (l16, g) element i: n = n0 + 16 nt + 4g + i, m = 16 mt + l16. The waves' partial
    // tiles are summed in wave order (XREG: in the slice order wave order gives the other forms,
    // slice (v + blk) mod 8 at position v), one (nt, mt) tile per wave; in GLU the gate tiles go
    // through LDS first and the up tiles second, and the wave holding gate tile (nt, mt) keeps
    // its bf16-rounded values for the product with up tile (nt, mt) of the second round.
    float gate[4] = {0.f, 0.f, 0.f, 0.f};
    if (NORM && !XREG) {  // row sums over the four g lanes (xor 16, 32: fixed order), one slot per wave
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            ss[mt] += __shfl_xor(ss[mt], 16);
            ss[mt] += __shfl_xor(ss[mt], 32);
            if (g == 0) lds.ss[wave][16 * mt + l16] = ss[mt];
        }
    }
#pragma unroll
    for (int round = 0; round < (GLU && !PAIR ? 2 : 1); ++round) {
        __syncthreads();  // every wave is done with its transpose region / the previous round
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                lds.acc[wave][nt * MT + mt][lane] = acc[round * NT + nt][mt];
        __syncthreads();
        for (int tile = wave; tile < NT * MT; tile += SG_WAVES) {
            const int rot = XREG ? blk % SG_WAVES : 0;
            sg_f32x4 t = lds.acc[rot][tile][lane];
#pragma unroll
            for (int v = 1; v < SG_WAVES; ++v) t += lds.acc[(v + rot) % SG_WAVES][tile][lane];
            const int nt = tile / MT, mt = tile % MT;
            const int m = 16 * mt + l16;
            if (NORM) {  // the row's sum of squares in wave order, then rstd (IEEE division, sqrt)
                float s = lds.ss[rot][m];
#pragma unroll
                for (int v = 1; v < SG_WAVES; ++v) s += lds.ss[(v + rot) % SG_WAVES][m];
                const float rstd = 1.0f / sqrtf(s / (float)K + eps);
#pragma unroll
                for (int i = 0; i < 4; ++i) t[i] *= rstd;
            }
            if (PAIR) {  // lanes g < 2 hold gate rows 4 g + i, lanes g + 2 their up rows
#pragma clang fp contract(off)
                float u[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    t[i] = bf16_to_f32(f32_to_bf16_rne(t[i]));
                    u[i] = __shfl_xor(t[i], 32);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {  // silu_mul's arithmetic: (g * (1 / (1 + e^-g))) * u
                    const float sg = 1.0f / (1.0f + expf(-t[i]));
                    t[i] = (t[i] * sg) * u[i];
                }
            } else if (GLU) {
#pragma clang fp contract(off)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v = bf16_to_f32(f32_to_bf16_rne(t[i]));
                    if (round == 0) {
                        gate[i] = v;
                    } else {  // silu_mul's arithmetic: (g * (1 / (1 + e^-g))) * u
                        const float sg = 1.0f / (1.0f + expf(-gate[i]));
                        t[i] = (gate[i] * sg) * v;
                    }
                }
                if (round == 0) continue;
            }
            if (m < M && (!(HALF || PAIR) || g < 2)) {
                // YFRAG: columns 8T + 4g .. + 4 (T = blk NT + nt) of row m are 8 bytes of lane
                // (16 (T mod 4) + l16) in block (T / 4) MT + mt
                const int T = blk * NT + nt;
                uint16_t* dst = YFRAG ? y + ((int64_t)(T / 4) * MT + mt) * 512 +
                                            8 * (16 * (T % 4) + l16) + 4 * g
                                      : y + (int64_t)m * ys + 4 * g +
                                            (PAIR ? 8 * T : n0 + 16 * nt);
                if (RES) {  // bf16(residual + bf16(sum)) in fp32, as add_rms_norm adds
                    const uint2 r = *reinterpret_cast<const uint2*>(dst);
                    const uint32_t rw[2] = {r.x, r.y};
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        t[i] = bf16_to_f32((uint16_t)(rw[i / 2] >> (16 * (i % 2)))) +
                               bf16_to_f32(f32_to_bf16_rne(t[i]));
                }
                *reinterpret_cast<uint2*>(dst) =
                    make_uint2(pack_bf16x2(t[0], t[1]), pack_bf16x2(t[2], t[3]));
                if (AMAX) {  // the stored (bf16) values, columns in increasing order
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float v = bf16_to_f32(f32_to_bf16_rne(t[i]));
                        const int n = n0 + 16 * nt + 4 * g + i;
                        if (amax_better(v, n, abv, abi)) {
                            abv = v;
                            abi = n;
                        }
                    }
                }
            }
        }
    }
    if (!LOOP || next >= nblk) break;
    __syncthreads();  // every wave is done reading the partial tiles before the next transposes
    blk = next;
    }
    if constexpr (AMAX) {
        __shared__ float s_bv[SG_WAVES][16];
        __shared__ int s_bi[SG_WAVES][16];
#pragma unroll
        for (int x = 16; x <= 32; x <<= 1) {  // the four g lanes of row 16 mt + l16
            const float ov = __shfl_xor(abv, x);
            const int oi = __shfl_xor(abi, x);
            if (amax_better(ov, oi, abv, abi)) {
                abv = ov;
                abi = oi;
            }
        }
        if (wave < NT * MT && g == 0) {  // wave w holds output tile w: (nt, mt) = (w / MT, w % MT)
            s_bv[wave][l16] = abv;
            s_bi[wave][l16] = abi;
        }
        __syncthreads();
        if (tid < M) {  // row m = tid: its tiles are nt MT + m / 16
            float v = -INFINITY;
            int i = 0x7fffffff;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int tile = nt * MT + tid / 16;
                if (amax_better(s_bv[tile][tid % 16], s_bi[tile][tid % 16], v, i)) {
                    v = s_bv[tile][tid % 16];
                    i = s_bi[tile][tid % 16];
                }
            }
            if (i != 0x7fffffff)  // a column was taken (any value but NaN)
                __hip_atomic_fetch_max(am.keys + tid, amax_key(v, i), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
        if (arrive_last(am.count, (int)(gridDim.x * gridDim.y * gridDim.z))) {
            if (tid < M) {  // the row's largest key; 0: no column taken (every value NaN)
                const uint64_t key = __hip_atomic_exchange(am.keys + tid, (uint64_t)0,
                                                           __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
                am.out[(int64_t)tid * am.os] =
                    key ? (int64_t)(0xffffffffu - (uint32_t)key) : (int64_t)0x7fffffff;
            }
            if (tid == 0) am.seed[0] += 1;
        }
    }
}

}  // namespace ie

using namespace ie;

// Argument checks shared by the entry points (n: weight rows).
static hipError_t skinny_check(const ie_bf16* x, int64_t x_stride, int32_t m, const ie_bf16* weight,
                               int64_t weight_stride, int32_t n, int32_t k, int32_t n_tiles,
                               const ie_bf16* y, int64_t y_stride) {
    IE_REQUIRE(x && weight && y, "null pointer");
    IE_REQUIRE(m <= 64, "at most 64 rows");
    IE_REQUIRE(n % 16 == 0 && k % (SG_WAVES * 32) == 0 && k > 0,
               "n must be a multiple of 16 and k of 256");
    IE_REQUIRE(n_tiles == 0 || n_tiles == 1 || n_tiles == 2 || n_tiles == 4,
               "n_tiles must be 0 (8-row tiles), 1, 2 or 4");
    IE_REQUIRE(n % (16 * std::max(1, n_tiles)) == 0, "n must be a multiple of 16 n_tiles");
    IE_REQUIRE(x_stride % 8 == 0 && weight_stride % 8 == 0 && y_stride % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(weight) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(y) & 7) == 0,
               "rows must be 16-byte aligned (8-byte for y)");
    IE_REQUIRE((int64_t)m * x_stride * 2 < (1LL << 31) &&
                   16LL * std::max(1, n_tiles) * weight_stride * 2 < (1LL << 31),
               "operands too large for 32-bit buffer offsets");
    return hipSuccess;
}

namespace {

struct SgCall {
    const uint16_t* x;
    int64_t xs;
    int m;
    const uint16_t* w;
    int64_t ws;
    int k;
    uint16_t* y;
    int64_t ys;
    int nh;
    float eps;
    int nblk;  // row blocks (the looping grid: more than its workgroups)
    SgAmax am;  // the greedy tokens (AMAX only)
};

template <int MT, int NT, int MODE>
void sg_go(dim3 grid, hipStream_t s, const SgCall& c) {
    hipLaunchKernelGGL((skinny_gemm_kernel<MT, NT, MODE>), grid, dim3(SG_THREADS), 0, s, c.x,
                       c.xs, c.m, c.w, c.ws, c.k, c.y, c.ys, c.nh, c.eps,
                       c.nblk > 0 ? c.nblk : (int)grid.x, c.am);
}

// One weight row block per workgroup: n_tiles 0 (8 rows), 1, 2 or 4 n-tiles of 16 rows (4 only
// where the LDS transpose region holds MT + 4 tiles; the caller has lowered n_tiles to fit).
template <int MT, int EXTRA>
void sg_rows(int n_tiles, dim3 grid, hipStream_t s, const SgCall& c) {
    switch (n_tiles) {
        case 0:
            if constexpr (!(EXTRA & SG_SWZ)) sg_go<MT, 1, SG_HALF | EXTRA>(grid, s, c);
            break;
        case 1: sg_go<MT, 1, EXTRA>(grid, s, c); break;
        case 2: sg_go<MT, 2, EXTRA>(grid, s, c); break;
        default:
            if constexpr (MT + 4 <= SG_MAX_TILES) sg_go<MT, 4, EXTRA>(grid, s, c);
            break;
    }
}

template <int EXTRA>
void sg_rows_mt(int mt, int n_tiles, dim3 grid, hipStream_t s, const SgCall& c) {
    switch (mt) {
        case 1: sg_rows<1, EXTRA>(n_tiles, grid, s, c); break;
        case 2: sg_rows<2, EXTRA>(n_tiles, grid, s, c); break;
        case 3: sg_rows<3, EXTRA>(n_tiles, grid, s, c); break;
        default: sg_rows<4, EXTRA>(n_tiles, grid, s, c); break;
    }
}

// The swizzled gate/up weight (paired tiles): n_tiles 1 ... 4 with MT + n_tiles <= 6.
template <int MT, int EXTRA>
void sg_pair_nt(int n_tiles, dim3 grid, hipStream_t s, const SgCall& c) {
    switch (n_tiles) {
        case 1: sg_go<MT, 1, SG_GLU | EXTRA>(grid, s, c); break;
        case 2: sg_go<MT, 2, SG_GLU | EXTRA>(grid, s, c); break;
        case 3:
            if constexpr (MT + 3 <= SG_MAX_TILES) sg_go<MT, 3, SG_GLU | EXTRA>(grid, s, c);
            break;
        default:
            if constexpr (MT + 4 <= SG_MAX_TILES) sg_go<MT, 4, SG_GLU | EXTRA>(grid, s, c);
            break;
    }
}

// Gate/up pairs: n_tiles 1 or 2 (2 only for MT <= 2, where the LDS region holds 2 + 2 + MT tiles);
// on the swizzled weight, sg_pair_nt.
template <int EXTRA>
void sg_glu_mt(int mt, int n_tiles, dim3 grid, hipStream_t s, const SgCall& c) {
    if constexpr (EXTRA & SG_SWZ) {
        switch (mt) {
            case 1: sg_pair_nt<1, EXTRA>(n_tiles, grid, s, c); break;
            case 2: sg_pair_nt<2, EXTRA>(n_tiles, grid, s, c); break;
            case 3: sg_pair_nt<3, EXTRA>(n_tiles, grid, s, c); break;
            default: sg_pair_nt<4, EXTRA>(n_tiles, grid, s, c); break;
        }
        return;
    }
    switch (mt) {
        case 1:
            if (n_tiles == 2) sg_go<1, 2, SG_GLU | EXTRA>(grid, s, c);
            else sg_go<1, 1, SG_GLU | EXTRA>(grid, s, c);
            break;
        case 2:
            if (n_tiles == 2) sg_go<2, 2, SG_GLU | EXTRA>(grid, s, c);
            else sg_go<2, 1, SG_GLU | EXTRA>(grid, s, c);
            break;
        case 3: sg_go<3, 1, SG_GLU | EXTRA>(grid, s, c); break;
        default: sg_go<4, 1, SG_GLU | EXTRA>(grid, s, c); break;
    }
}

template <int EXTRA>
void sg_dispatch(bool glu, int mt, int n_tiles, dim3 grid, hipStream_t s, const SgCall& c) {
    if constexpr (!(EXTRA & SG_RES)) {  // the residual form has no gate/up variant
        if (glu) {
            sg_glu_mt<EXTRA>(mt, n_tiles, grid, s, c);
            return;
        }
    }
    if constexpr (!(EXTRA & SG_YFRAG)) sg_rows_mt<EXTRA>(mt, n_tiles, grid, s, c);
}

}  // namespace

extern "C" hipError_t ie_skinny_gemm_fused(const ie_bf16* x, int64_t x_stride, int32_t m,
                                           const ie_bf16* weight, int64_t weight_stride,
                                           int32_t n, int32_t k, int32_t n_tiles, int32_t flags,
                                           float eps, ie_bf16* y, int64_t y_stride,
                                           hipStream_t stream) {
    IE_REQUIRE(m >= 0 && n >= 0 && k >= 0, "negative sizes");
    const int form = flags & ~(IE_SKINNY_SWIZZLED | IE_SKINNY_X_FRAGMENTS | IE_SKINNY_Y_FRAGMENTS);
    IE_REQUIRE(form == 0 || form == IE_SKINNY_NORM || form == IE_SKINNY_SILU_MUL ||
                   form == (IE_SKINNY_NORM | IE_SKINNY_SILU_MUL) || form == IE_SKINNY_RESIDUAL,
               "flags: 0, NORM, SILU_MUL, NORM | SILU_MUL or RESIDUAL, each optionally | SWIZZLED");
    const bool norm = flags & IE_SKINNY_NORM, glu = flags & IE_SKINNY_SILU_MUL,
               res = flags & IE_SKINNY_RESIDUAL, swz = flags & IE_SKINNY_SWIZZLED,
               xfrag = flags & IE_SKINNY_X_FRAGMENTS;
    IE_REQUIRE(!xfrag || ((form == 0 || form == IE_SKINNY_RESIDUAL) && x_stride == k),
               "x in fragment order: the plain or residual form, x_stride k");
    const bool yfrag = flags & IE_SKINNY_Y_FRAGMENTS;
    IE_REQUIRE(!yfrag || (glu && swz && n % 64 == 0 && y_stride == n / 2),
               "y in fragment order: the swizzled gate/up form, n / 2 a multiple of 32, "
               "y_stride n / 2");
    IE_REQUIRE(!norm || (eps >= 0.f && eps < 1e30f), "eps must be finite and >= 0");
    IE_REQUIRE(!swz || (n_tiles >= 1 && weight_stride == k),
               "a swizzled weight takes the n_tiles (1, 2 or 4; 1 ... 4 for the gate/up form) it "
               "was swizzled for and weight_stride k");
    IE_REQUIRE(n_tiles != 3 || (glu && swz),
               "n_tiles must be 0, 1, 2 or 4 (3: only the swizzled gate/up form)");
    if (m == 0 || n == 0) return hipSuccess;
    if (glu && swz) {
        IE_REQUIRE(n_tiles <= 4 && n % 2 == 0 && (n / 2) % (8 * n_tiles) == 0,
                   "n must be even and n / 2 a multiple of 8 n_tiles (n_tiles 1 ... 4)");
    } else if (glu) {
        IE_REQUIRE(n_tiles == 1 || n_tiles == 2, "n_tiles must be 1 or 2");
        IE_REQUIRE(n % 2 == 0 && (n / 2) % (16 * n_tiles) == 0,
                   "n must be even and n / 2 a multiple of 16 n_tiles");
    }
    hipError_t e = skinny_check(x, x_stride, m, weight, weight_stride, n, k,
                                n_tiles == 3 ? 1 : n_tiles, y, y_stride);
    if (e != hipSuccess) return e;
    const int mt = (m + 15) / 16;
    SgCall c{(const uint16_t*)x, x_stride, m, (const uint16_t*)weight, weight_stride, k,
             (uint16_t*)y, y_stride, glu ? n / 2 : 0, eps, 0};
    dim3 grid;
    IE_REQUIRE(!swz || n_tiles + mt <= SG_MAX_TILES,
               "a swizzled weight's n_tiles is too wide for this many rows (its layout depends "
               "on n_tiles, which cannot be lowered)");
    if (glu && swz) {  // paired tiles: 8 output columns each
        grid = dim3((unsigned)(n / 2 / (8 * n_tiles)));
    } else if (glu) {
        // gate and up tiles: lowered to one n-tile where m leaves too little LDS for two
        if (2 * n_tiles + mt > SG_MAX_TILES) n_tiles = 1;
        grid = dim3((unsigned)(n / 2 / (16 * n_tiles)));
    } else {
        // n_tiles is a performance choice: it is lowered until the LDS transpose region fits
        while (n_tiles > 1 && n_tiles + mt > SG_MAX_TILES) n_tiles >>= 1;
        grid = dim3((unsigned)(n_tiles == 0 ? n / 8 : n / (16 * n_tiles)));
    }
    const int mode = (norm ? SG_NORM : 0) | (res ? SG_RES : 0);
#define IE_SG_DISPATCH(SW)                                                                 \
    switch (mode) {                                                                        \
        case SG_NORM: sg_dispatch<SG_NORM | SW>(glu, mt, n_tiles, grid, stream, c); break; \
        case SG_RES: sg_dispatch<SG_RES | SW>(false, mt, n_tiles, grid, stream, c); break; \
        default: sg_dispatch<SG_PLAIN | SW>(glu, mt, n_tiles, grid, stream, c); break;     \
    }
    if (yfrag) {
        if (norm) sg_dispatch<SG_NORM | SG_SWZ | SG_YFRAG>(true, mt, n_tiles, grid, stream, c);
        else sg_dispatch<SG_SWZ | SG_YFRAG>(true, mt, n_tiles, grid, stream, c);
    } else if (xfrag) {
        if (swz) {
            if (res) sg_rows_mt<SG_RES | SG_SWZ | SG_XFRAG>(mt, n_tiles, grid, stream, c);
            else sg_rows_mt<SG_SWZ | SG_XFRAG>(mt, n_tiles, grid, stream, c);
        } else {
            if (res) sg_rows_mt<SG_RES | SG_XFRAG>(mt, n_tiles, grid, stream, c);
            else sg_rows_mt<SG_XFRAG>(mt, n_tiles, grid, stream, c);
        }
    } else if (swz && !glu && (mode == 0 || (mode == SG_NORM && k == SG_XREG_K)) && n_tiles > 0 &&
               (int)grid.x > 4 * device_cu_count()) {
        // a weight of many more row blocks than CUs (the LM head): one looping workgroup per CU
        c.nblk = (int)grid.x;
        const dim3 cus((unsigned)device_cu_count());
        if (mode == SG_NORM)
            sg_rows_mt<SG_NORM | SG_SWZ | SG_LOOP | SG_XREG>(mt, n_tiles, cus, stream, c);
        else if (k == SG_XREG_K)
            sg_rows_mt<SG_SWZ | SG_LOOP | SG_XREG>(mt, n_tiles, cus, stream, c);
        else
            sg_rows_mt<SG_SWZ | SG_LOOP>(mt, n_tiles, cus, stream, c);
    } else if (swz) {
        IE_SG_DISPATCH(SG_SWZ)
    } else {
        IE_SG_DISPATCH(0)
    }
#undef IE_SG_DISPATCH
    return hipGetLastError();
}

// The LM head with the greedy tokens (AMAX): the looping form of ie_skinny_gemm_fused, plain or
// NORM, over a weight swizzled for n_tiles, plus tokens[m] and the seed advanced by one.
constexpr int SG_AMAX_ROWS = 64;
extern "C" size_t ie_skinny_lm_head_greedy_workspace_size(void) {
    return SG_AMAX_ROWS * sizeof(uint64_t) + 256;  // the row maxima, then the count
}

extern "C" hipError_t ie_skinny_lm_head_greedy(
    const ie_bf16* x, int64_t x_stride, int32_t m, const ie_bf16* weight, int32_t n, int32_t k,
    int32_t n_tiles, int32_t flags, float eps, ie_bf16* logits, int64_t logits_stride,
    int64_t* tokens, int64_t tokens_stride, int64_t* seed, void* workspace,
    size_t workspace_bytes, hipStream_t stream) {
    IE_REQUIRE(m >= 0 && n >= 0 && k >= 0, "negative sizes");
    IE_REQUIRE(flags == 0 || flags == IE_SKINNY_NORM, "flags: 0 or NORM");
    IE_REQUIRE(flags == 0 || (eps >= 0.f && eps < 1e30f), "eps must be finite and >= 0");
    IE_REQUIRE(n_tiles == 1 || n_tiles == 2 || n_tiles == 4, "n_tiles must be 1, 2 or 4");
    if (m == 0) return hipSuccess;
    IE_REQUIRE(n > 0 && k == SG_XREG_K, "the looping LM head form: k 2048");
    IE_REQUIRE(tokens && seed && workspace, "null pointer");
    IE_REQUIRE(workspace_bytes >= ie_skinny_lm_head_greedy_workspace_size() &&
                   (reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
               "workspace too small or misaligned");
    hipError_t e = skinny_check(x, x_stride, m, weight, k, n, k, n_tiles, logits, logits_stride);
    if (e != hipSuccess) return e;
    const int mt = (m + 15) / 16;
    IE_REQUIRE(n_tiles + mt <= SG_MAX_TILES, "n_tiles too wide for this many rows");
    SgCall c{(const uint16_t*)x, x_stride, m, (const uint16_t*)weight, k, k,
             (uint16_t*)logits, logits_stride, 0, eps, n / (16 * n_tiles)};
    c.am = SgAmax{reinterpret_cast<uint64_t*>(workspace),
                  reinterpret_cast<uint32_t*>(reinterpret_cast<uint64_t*>(workspace) +
                                              SG_AMAX_ROWS),
                  tokens, tokens_stride, seed};
    const dim3 grid((unsigned)std::min(c.nblk, device_cu_count()));
    if (flags == IE_SKINNY_NORM)
        sg_rows_mt<SG_NORM | SG_SWZ | SG_LOOP | SG_XREG | SG_AMAX>(mt, n_tiles, grid, stream, c);
    else
        sg_rows_mt<SG_SWZ | SG_LOOP | SG_XREG | SG_AMAX>(mt, n_tiles, grid, stream, c);
    return hipGetLastError();
}

// The fragment order of the SWZ form for n_tiles G: the 1 KB block of 16-row group R and
// 32-column step S, at block index ((R / G) * k / 32 + S) * G + R % G, holds, at 16 bytes per
// lane L = 16 g + r, weight row 16 R + r, columns 32 S + 8 g .. + 8. One wave per block.
// pair: the gate/up weight (n / 2 gate rows, then the up rows) in paired order, 16-row tile R
// holding gate rows [8 R, +8) then up rows [n / 2 + 8 R, +8).
__global__ __launch_bounds__(256) void skinny_weight_swizzle_kernel(const uint16_t* __restrict__ w,
                                                                    int64_t ws, int n, int k,
                                                                    int G, int pair,
                                                                    uint16_t* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t steps = k / 32;
    if (blk >= (int64_t)(n / 16) * steps) return;
    const int64_t R = blk / steps, S = blk % steps;
    const int r = lane & 15, g = lane >> 4;
    const int64_t row = !pair ? 16 * R + r : r < 8 ? 8 * R + r : n / 2 + 8 * R + r - 8;
    const uint4 v = *reinterpret_cast<const uint4*>(w + row * ws + 32 * S + 8 * g);
    const int64_t dst = ((R / G) * steps + S) * G + R % G;
    *reinterpret_cast<uint4*>(out + dst * 512 + 8 * lane) = v;
}

static hipError_t weight_swizzle(const ie_bf16* weight, int64_t weight_stride, int32_t n,
                                 int32_t k, int32_t n_tiles, bool pair, ie_bf16* out,
                                 hipStream_t stream) {
    IE_REQUIRE(n >= 0 && k >= 0, "negative sizes");
    if (pair) IE_REQUIRE(n_tiles >= 1 && n_tiles <= 4, "n_tiles must be 1, 2, 3 or 4");
    else IE_REQUIRE(n_tiles == 1 || n_tiles == 2 || n_tiles == 4, "n_tiles must be 1, 2 or 4");
    if (n == 0 || k == 0) return hipSuccess;
    IE_REQUIRE(weight && out, "null pointer");
    IE_REQUIRE(n % (16 * n_tiles) == 0 && k % 32 == 0,
               "n must be a multiple of 16 n_tiles and k of 32");
    IE_REQUIRE(weight_stride >= k && weight_stride % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(weight) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "rows must be 16-byte aligned");
    const int64_t blocks = (int64_t)(n / 16) * (k / 32);
    hipLaunchKernelGGL(skinny_weight_swizzle_kernel, dim3((unsigned)((blocks + 3) / 4)),
                       dim3(256), 0, stream, (const uint16_t*)weight, weight_stride, n, k,
                       (int)n_tiles, pair ? 1 : 0, (uint16_t*)out);
    return hipGetLastError();
}

extern "C" hipError_t ie_skinny_weight_swizzle(const ie_bf16* weight, int64_t weight_stride,
                                               int32_t n, int32_t k, int32_t n_tiles,
                                               ie_bf16* out, hipStream_t stream) {
    return weight_swizzle(weight, weight_stride, n, k, n_tiles, false, out, stream);
}

extern "C" hipError_t ie_skinny_weight_swizzle_gate_up(const ie_bf16* weight,
                                                       int64_t weight_stride, int32_t n,
                                                       int32_t k, int32_t n_tiles, ie_bf16* out,
                                                       hipStream_t stream) {
    return weight_swizzle(weight, weight_stride, n, k, n_tiles, true, out, stream);
}

extern "C" hipError_t ie_skinny_gemm(const ie_bf16* x, int64_t x_stride, int32_t m,
                                     const ie_bf16* weight, int64_t weight_stride, int32_t n,
                                     int32_t k, int32_t n_tiles, ie_bf16* y, int64_t y_stride,
                                     hipStream_t stream) {
    return ie_skinny_gemm_fused(x, x_stride, m, weight, weight_stride, n, k, n_tiles, 0, 0.f, y,
                                y_stride, stream);
}

extern "C" hipError_t ie_skinny_gemm_silu_mul(const ie_bf16* x, int64_t x_stride, int32_t m,
                                              const ie_bf16* weight, int64_t weight_stride,
                                              int32_t n, int32_t k, int32_t n_tiles, ie_bf16* y,
                                              int64_t y_stride, hipStream_t stream) {
    return ie_skinny_gemm_fused(x, x_stride, m, weight, weight_stride, n, k, n_tiles,
                                IE_SKINNY_SILU_MUL, 0.f, y, y_stride, stream);
}
