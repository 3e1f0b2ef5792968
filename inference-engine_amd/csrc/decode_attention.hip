// Split-K GQA decode attention over the int8 KV cache, for gfx950.
//
// Work split (same rule as qwen3-1.7b/kernels.py:20-70): every decoding sequence's tokens
// [0, cached_len + 1) are cut into pieces of `piece` tokens, piece = roundup(max(MIN_PIECE,
// cdiv(total_tokens, TARGET)), MIN_PIECE) with TARGET = CUs * WG_PER_CU / Hkv workgroups per KV
// head (when B <= TARGET the piece is grown until the pieces fit TARGET, see decode_piece). The
// pieces of all sequences form one work list; workgroup (w, kv head) takes entry w. The grid is
// (TARGET, Hkv) when B <= TARGET, else (TARGET + B, Hkv): it depends on shapes only, so the
// launch is graph-capturable, and each workgroup finds its (sequence, piece) on the device from
// cached_lens.
//
// One workgroup = 8 waves = one (sequence, piece, kv head), i.e. both query heads of the GQA
// pair. Lane (g, c) of a wave (g = lane / 8, c = lane % 8) owns channels [16c, 16c+16) of the
// four tokens 4g..4g+3 of the wave's 32-token block: each K and V row (128 int8) is read by 8
// lanes with 16-byte loads, so one load instruction of a wave covers 8 full 128-byte rows.
//
// Arithmetic (all VALU, no MFMA: the op is HBM-bound):
//   int8 -> fp16 by byte permute into the fp16 pattern 0x64xx (= 1024 + byte) after flipping
//   the sign bit, i.e. the fp16 value 1152 + x exactly; the 1152 offset is removed once per
//   score (q . 1152 = 1152 * sum(q)) and once per output (sum of P).
//   q is scaled by a power of two per head so it is exact in fp16; QK^T and PV use the
//   fp32-accumulating v_dot2_f32_f16. QK partial dots are reduced across the 8 lanes of a row
//   with DPP. Online softmax in base 2 per lane group; groups and waves are merged at the end
//   (log-sum-exp), then either the output is written (one piece) or fp32 partials (m, l, acc)
//   go to the workspace and the sequence's last piece to finish merges them (the reference's
//   combine kernel, kernels.py:216-264, folded into the same launch).
#include <mutex>

#include "ie_common.h"
#include "kv_math.h"

// Launch shape: 16 waves per CU (the 128-register budget allows 4 waves per SIMD), as 8-wave
// workgroups, 2 per CU, while the batch fits their per-head target, else 4-wave workgroups
// (4 per CU) or 2-wave workgroups (8 per CU), whose targets are twice and four times as large
// (decode_waves). Measured on MI355X: 8 waves are best up to B = 64 (one 4096-token piece per
// row at B=64 ctx=4096); above, the smaller workgroups keep every sequence in one resident
// round of fitted pieces instead of the reference rule's target + B pieces: B=96 ctx=1024
// -15 % (4 waves), B=256 ctx=512 -31 % and ctx=1024 -11 % (2 waves), long contexts level.

namespace ie {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// K/V/scale loads carry the non-temporal cache policy (aux bit 1, "nt" on gfx94x/gfx950): every
// byte is read once, and streaming it past the caches raised read bandwidth from ~6.0 to
// ~7.0 TB/s in isolation.
#ifndef IE_DECODE_HEAD_FAST_MIN_BATCH
#define IE_DECODE_HEAD_FAST_MIN_BATCH 0
#endif
#ifndef IE_DECODE_LOAD_AUX
#define IE_DECODE_LOAD_AUX 2
#endif

constexpr int DA_WAVES_PER_CU = 16;
constexpr int DA_U = 4;                // tokens per lane group per block
constexpr int DA_TOK_WAVE = 8 * DA_U;  // 32 tokens per wave block
constexpr int DA_MIN_PIECE = 128;
constexpr int DA_MAX_SPLITS = 1024;  // per-KV-head workgroup target, at most
constexpr int DA_D = 128;
constexpr uint32_t K64 = 0x64646464u;
constexpr float OFFSET = 1152.0f;  // fp16(0x64xx) = 1024 + byte, byte = x + 128


// Workgroup target per unit (KV head x query-head pair; the KV head at GQA 2) of workgroups of
// `waves` waves: one resident round.
int decode_target(int units, int waves) {
    return std::min(DA_MAX_SPLITS, std::max(1, device_cu_count() * (DA_WAVES_PER_CU / waves) /
                                                   std::max(1, units)));
}
// Waves per workgroup for a batch: the largest workgroup whose target holds the batch, else
// the smallest.
int decode_waves(int batch, int units) {
    for (int w = 8; w > 2; w /= 2)
        if (batch <= decode_target(units, w)) return w;
    return 2;
}
// Units of a launch: KV heads x query-head pairs per KV head.
int decode_units(int hq, int hkv) { return hkv * ((hq / std::max(1, hkv) + 1) / 2); }


// Piece size for this step; wave-uniform, every lane returns it. The reference's rule
// (kernels.py:20-37) gives p0 = roundup(max(128, cdiv(total, target)), 128), but every sequence
// rounds its own split count up, so its pieces can number up to target + nd and spill past the
// one resident wave of workgroups that target sizes. When nd <= target the piece is instead the
// smallest multiple of 128, at least p0, whose pieces number at most target: a binary search,
// since the count falls as the piece grows and is nd at the longest sequence's length.
// n0: this lane's n_b of the first 64 sequences (0 past nd).
__device__ int decode_piece(const int32_t* __restrict__ cached_lens, int nd, int target, int n0) {
    const int lane = threadIdx.x & 63;
    auto n_of = [&](int b0) { return b0 == 0 ? n0 : (b0 + lane < nd ? cached_lens[b0 + lane] + 1 : 0); };
    int total = 0, longest = 0;
    for (int b0 = 0; b0 < nd; b0 += 64) {
        const int n = n_of(b0);
        total += wave_sum_i(n);
        longest = max(longest, (int)wave_max((float)n));
    }
    const int k0 = max(1, cdiv_i(cdiv_i(total, target), DA_MIN_PIECE));
    if (nd > target) return k0 * DA_MIN_PIECE;
    auto pieces = [&](int k) {
        const Divisor p = divisor(k * DA_MIN_PIECE);
        int c = 0;
        for (int b0 = 0; b0 < nd; b0 += 64) c += wave_sum_i(div_ceil(n_of(b0), p));
        return c;
    };
    int lo = k0, hi = max(k0, cdiv_i(longest, DA_MIN_PIECE));  // pieces(hi) <= nd <= target
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (pieces(mid) <= target) hi = mid;
        else lo = mid + 1;
    }
    return lo * DA_MIN_PIECE;
}

struct Work {
    int b, split, needed, piece;
};

// Entry `w` of the work list (kernels.py:40-70); needed == 0 for idle workgroups. `raw0`: this
// lane's cached_lens entry of the first 64 sequences, loaded by the caller bounded by the batch
// size instead of num_decoding, so that it shares one memory round trip with num_decoding.
__device__ Work decode_assign(const int32_t* __restrict__ cached_lens, int nd, int w, int target,
                              int raw0) {
    const int lane = threadIdx.x & 63;
    const int n0 = lane < nd ? raw0 + 1 : 0;
    Work r{0, 0, 0, decode_piece(cached_lens, nd, target, n0)};
    int before = 0;
    for (int b0 = 0; b0 < nd; b0 += 64) {
        const int b = b0 + lane;
        const int s = b < nd ? cdiv_i(b0 == 0 ? n0 : cached_lens[b] + 1, r.piece) : 0;
        const int incl = wave_incl_scan_i(s) + before;
        const int excl = incl - s;
        const unsigned long long hit = __ballot(s > 0 && excl <= w && w < incl);
        if (hit) {
            const int src = __ffsll((long long)hit) - 1;  // wave-uniform
            r.b = b0 + src;
            r.split = w - __builtin_amdgcn_readlane(excl, src);
            r.needed = __builtin_amdgcn_readlane(s, src);
            return r;
        }
        before = __builtin_amdgcn_readlane(incl, 63);
    }
    return r;
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
// The lane's index in its wave, from the lane-count instructions: with the wave index (uniform)
// it rebuilds the thread index after the block loop, so that no register holds it there.
__device__ __forceinline__ int lane_id() {
    return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}
__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ float fdot2(half2_t a, half2_t b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}
__device__ __forceinline__ float exp2_safe(float x) { return __builtin_amdgcn_exp2f(x); }

struct DecodeArgs {
    const uint16_t* q;
    int64_t q_sb, q_sh;
    ie_kv_cache c;
    const int32_t* cached_lens;
    const int32_t* slot_ids;
    const int32_t* num_decoding;
    float scale_log2;  // softmax scale * log2(e)
    uint16_t* out;
    int64_t o_sb, o_sh;
    float* part_acc;     // [Hq, nwork, 128]: work entry w's partial output for query head h
    float* part_m;       // [Hq, nwork]
    float* part_l;       // [Hq, nwork]
    uint32_t* arrivals;  // [B, Hkv]: pieces of the sequence done; 0 between calls
    // The work list precomputed for this step (ie_decode_attention_plan: row w = (b, split,
    // needed, piece) of workgroup index w), or null: every workgroup derives its entry itself.
    const int32_t* plan;
    int target, nwork, hq, hkv;
    int ratio;   // query heads per KV head (GQA ratio, 1 ... 16)
    int npairs;  // query-head pairs per KV head, cdiv(ratio, 2): a workgroup serves one pair
    int units;   // hkv * npairs: the grid's second dimension
    int batch;        // rows of q / cached_lens (num_decoding[0] <= batch)
    int head_fast;    // 1: grid (Hkv, pieces), the KV head in blockIdx.x; 0: grid (pieces, Hkv)
    // The fused form (ie_decode_attention_rope): q holds the QKV projection's raw rows, and the
    // launch does fused_rope_kv_decode's work itself: q normed, rotated and scaled by the
    // calibration as that kernel computes it, and the new token's K/V row quantized and written
    // to the cache by the piece that ends at it.
    const uint16_t* k_new;
    int64_t k_sb, k_sh;
    const uint16_t* v_new;
    int64_t v_sb, v_sh;
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    const uint16_t* cos;
    const uint16_t* sin;
    int64_t cos_sb, sin_sb;
    float eps;
};

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4u ld128(rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, IE_DECODE_LOAD_AUX);
}

// Running softmax state of one lane: query heads (2hk, 2hk+1), channels [16c, 16c+16).
// The PV products are fp16 values of p * v_scale * 2^ve: the exponent ve is chosen from the V
// scales the lane group has seen so that the largest product stays inside fp16's normal range
// whatever the magnitude of V (the reference rounds p * v_scale to bf16, whose exponent range
// is fp32's). l, ps and acc all carry the factor 2^ve, so the state is an ordinary online
// softmax whose running maximum m is kept as (max score - ve), and it merges as one.
struct LaneState {
    float m[2], l[2], ps[2];
    float acc[2][16];
    float ve;       // an integer
    uint32_t vlo;   // bits of 2^(8 - ve): the V scales this ve serves are [2^(8-ve), 2^(15-ve))
};

// Registers of one 32-token block of a wave: lane group g holds tokens t0+4g .. t0+4g+3,
// channels [16c, 16c+16), plus their 4 K (or V) scales.
struct KVRegs {
    v4u x[DA_U];
    v4u scale;
};

__device__ __forceinline__ void load_block(KVRegs& r, rsrc_t rows, rsrc_t scales, int tok,
                                           int cc) {
    const int off = tok * DA_D + 16 * cc;
#pragma unroll
    for (int u = 0; u < DA_U; ++u) r.x[u] = ld128(rows, off + u * DA_D);
    r.scale = ld128(scales, tok * 4);
}

// Scores of the block in base 2 up to the head's factor kmul (applied in block_pv):
// t = (q.k - 1152 sum q) * k_scale, where q is q * 2^e in fp16 and kmul = scale * log2(e) / 2^e.
// The 1152 sum q offset enters as the dot chain's starting value: qoff = -1152 sum q / 8 in
// each of the 8 lanes of a row, which the row sum adds up. qoff and kmul are wave-uniform.
// With MASKED, tokens at or past t_end score -inf (their loads returned zeros: buffer range).
template <bool MASKED>
__device__ __forceinline__ void block_scores(float (&t)[DA_U][2], const KVRegs& k,
                                             const half2_t (&qh)[2][8], const float (&qoff)[2],
                                             int tok, int t_end) {
#pragma unroll
    for (int u = 0; u < DA_U; ++u) {
        float d0 = qoff[0], d1 = qoff[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t x = k.x[u][i] ^ 0x80808080u;
            const half2_t h01 = as_h2(__builtin_amdgcn_perm(K64, x, 0x04010400u));
            const half2_t h23 = as_h2(__builtin_amdgcn_perm(K64, x, 0x04030402u));
            d0 = fdot2(qh[0][2 * i], h01, d0);
            d0 = fdot2(qh[0][2 * i + 1], h23, d0);
            d1 = fdot2(qh[1][2 * i], h01, d1);
            d1 = fdot2(qh[1][2 * i + 1], h23, d1);
        }
        d0 = sum8(d0);
        d1 = sum8(d1);
        const float ks = __uint_as_float(k.scale[u]);
        t[u][0] = d0 * ks;
        t[u][1] = d1 * ks;
        if (MASKED && tok + u >= t_end) t[u][0] = t[u][1] = -INFINITY;
    }
}

// Online-softmax update of the lane group and the PV accumulation of the block; scores are
// s = t * kmul (kmul > 0).
__device__ __forceinline__ void block_pv(LaneState& st, const float (&t)[DA_U][2],
                                         const KVRegs& v, const float (&kmul)[2]) {
    // The block's largest V scale vmax lies in [2^(ex-1), 2^ex). With p <= 2^ve the products
    // stay below 2^15 while vmax < 2^(15-ve); the exponent is re-chosen (ve = 15 - ex, so
    // vmax * 2^ve lies in [2^14, 2^15)) when that fails, or when vmax < 2^(8-ve), i.e. the
    // scales fell by 2^6 or more and small products would lose precision. Both bounds are one
    // unsigned compare on the float bits. The state is rescaled by the exact power of two and
    // m moves with ve. Scales past the piece's end load as 0 and change nothing.
    const float vmax = fmaxf(fmaxf(__uint_as_float(v.scale[0]), __uint_as_float(v.scale[1])),
                             fmaxf(__uint_as_float(v.scale[2]), __uint_as_float(v.scale[3])));
    if (__float_as_uint(vmax) - st.vlo >= (7u << 23)) {
        if (vmax > 0.0f) {
            const int ex = __builtin_amdgcn_frexp_expf(vmax);
            const float ve = (float)(15 - ex);
            const float d = ve - st.ve;
            const float r = ldexpf(1.0f, (int)d);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int j = 0; j < 16; ++j) st.acc[h][j] *= r;
                st.l[h] *= r;
                st.ps[h] *= r;
                st.m[h] -= d;  // -inf stays -inf
            }
            st.ve = ve;
            st.vlo = (uint32_t)(ex - 7 + 127) << 23;
        }
    }
    float nms[2];  // minus the effective running max, the exp2 argument's offset
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float mt =
            fmaxf(fmaxf(t[0][h], t[1][h]), fmaxf(t[2][h], t[3][h])) * kmul[h] - st.ve;
        if (mt > st.m[h]) {
            const float alpha = exp2_safe(st.m[h] - mt);  // m = -inf -> 0
#pragma unroll
            for (int j = 0; j < 16; ++j) st.acc[h][j] *= alpha;
            st.l[h] *= alpha;
            st.ps[h] *= alpha;
            st.m[h] = mt;
        }
        // p = 2^(s - max + ve) <= 2^ve
        nms[h] = st.m[h] == -INFINITY ? 0.0f : -st.m[h];
    }
    half2_t pp[DA_U / 2][2];  // (p * v_scale * 2^ve) of token pairs, fp16
#pragma unroll
    for (int pr = 0; pr < DA_U / 2; ++pr)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float pa = exp2_safe(__builtin_fmaf(t[2 * pr][h], kmul[h], nms[h]));
            const float pb = exp2_safe(__builtin_fmaf(t[2 * pr + 1][h], kmul[h], nms[h]));
            st.l[h] += pa + pb;
            pp[pr][h] = half2_t{(_Float16)(pa * __uint_as_float(v.scale[2 * pr])),
                                (_Float16)(pb * __uint_as_float(v.scale[2 * pr + 1]))};
            st.ps[h] = fdot2(pp[pr][h], half2_t{(_Float16)1.0f, (_Float16)1.0f}, st.ps[h]);
        }
#pragma unroll
    for (int pr = 0; pr < DA_U / 2; ++pr) {
        const int ua = 2 * pr, ub = ua + 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t xa = v.x[ua][i] ^ 0x80808080u, xb = v.x[ub][i] ^ 0x80808080u;
            const uint32_t t01 = __builtin_amdgcn_perm(xb, xa, 0x05010400u);
            const uint32_t t23 = __builtin_amdgcn_perm(xb, xa, 0x07030602u);
            const half2_t c[4] = {as_h2(__builtin_amdgcn_perm(K64, t01, 0x04010400u)),
                                  as_h2(__builtin_amdgcn_perm(K64, t01, 0x04030402u)),
                                  as_h2(__builtin_amdgcn_perm(K64, t23, 0x04010400u)),
                                  as_h2(__builtin_amdgcn_perm(K64, t23, 0x04030402u))};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                st.acc[0][4 * i + j] = fdot2(pp[pr][0], c[j], st.acc[0][4 * i + j]);
                st.acc[1][4 * i + j] = fdot2(pp[pr][1], c[j], st.acc[1][4 * i + j]);
            }
        }
    }
}

#ifndef IE_DECODE_WAVES_PER_EU
#define IE_DECODE_WAVES_PER_EU 4
#endif

// GQA2: the launch's GQA ratio is 2 (one query-head pair per KV head), so the pair's query
// heads are 2 hk and 2 hk + 1 at compile time; other ratios take the generic form.
template <int WAVES, bool ROPE, bool GQA2>
__global__ __launch_bounds__(WAVES * IE_WAVE)
__attribute__((amdgpu_waves_per_eu(IE_DECODE_WAVES_PER_EU))) void decode_attention_kernel(
    DecodeArgs a) {
    constexpr int THREADS = WAVES * IE_WAVE;
    constexpr int TOK_WG = WAVES * DA_TOK_WAVE;  // tokens per workgroup step
    const int lane0 = threadIdx.x & 63;
    // The first 64 sequences' lengths and cache slots, issued beside num_decoding: for them the
    // row to stream is known from registers once the work entry is found.
    const int raw0 = lane0 < a.batch ? a.cached_lens[lane0] : 0;
    const int slot0 = lane0 < a.batch ? a.slot_ids[lane0] : 0;
    const int nd = a.num_decoding[0];
    // the workgroup's (KV head, query-head pair): query heads qh0 = ratio * hk + 2 * pair and
    // qh0 + 1 (the pair of an odd ratio's last pair is one head: has2 = false)
    const int hk = a.head_fast ? blockIdx.x : blockIdx.y;
    const int pair = GQA2 ? 0 : (int)blockIdx.z;
    const int item = a.head_fast ? blockIdx.y : blockIdx.x;
    const int unit = GQA2 ? hk : hk * a.npairs + pair;
    const int qh0 = GQA2 ? 2 * hk : uniform(a.ratio * hk + 2 * pair);
    const bool has2 = GQA2 || 2 * pair + 1 < a.ratio;
    const int qh1 = has2 ? qh0 + 1 : qh0;  // an absent second head repeats the first
    Work wk;
    if (a.plan) {  // one 16-byte row, requested with the loads above
        const int4 r = *reinterpret_cast<const int4*>(a.plan + 4 * item);
        wk = Work{r.x, r.y, r.z, r.w};
    } else {
        wk = decode_assign(a.cached_lens, nd, item, a.target, raw0);
    }
    // Wave-uniform by construction; readfirstlane lets the compiler keep them (and the buffer
    // descriptors built from them) in SGPRs.
    wk.needed = uniform(wk.needed);
    if (wk.needed == 0) return;
    const int b = uniform(wk.b);
    const int split = uniform(wk.split);
    const int piece = uniform(wk.piece);
    const int n_end =
        b < 64 ? __builtin_amdgcn_readlane(raw0, b) + 1 : uniform(a.cached_lens[b] + 1);
    const int t_begin = split * piece;
    const int slot = b < 64 ? __builtin_amdgcn_readlane(slot0, b) : uniform(a.slot_ids[b]);
    // In the fused form the piece that ends at the new token (the sequence's last) takes that
    // token from registers, not from the cache it writes it to: it streams one token less.
    const bool last = ROPE && split == wk.needed - 1;
    const int t_end = min(t_begin + piece, n_end) - (last ? 1 : 0);

    const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
    const int g = lane >> 3, cc = lane & 7;

    // Buffer resources over this (slot, kv head) row, bounded at the piece's end.
    const int8_t* krow = a.c.k + slot * a.c.stride_slot + hk * a.c.stride_head;
    const int8_t* vrow = a.c.v + slot * a.c.stride_slot + hk * a.c.stride_head;
    const float* ksrow = a.c.k_scale + slot * a.c.scale_stride_slot + hk * a.c.scale_stride_head;
    const float* vsrow = a.c.v_scale + slot * a.c.scale_stride_slot + hk * a.c.scale_stride_head;
    const rsrc_t rk = make_rsrc(krow, (uint32_t)t_end * DA_D);
    const rsrc_t rv = make_rsrc(vrow, (uint32_t)t_end * DA_D);
    const rsrc_t rks = make_rsrc(ksrow, (uint32_t)t_end * 4);
    const rsrc_t rvs = make_rsrc(vsrow, (uint32_t)t_end * 4);

    // ---- q of the two heads of this KV head, channels [16cc, 16cc + 16) ----
    half2_t qh[2][8];
    float qoff[2], kmul[2];  // wave-uniform (kept in SGPRs)
    uint4 qraw[2][2];
    // Fused form, in fused_rope_kv_decode's layout (lane i holds channels i and i + 64): every
    // wave norms and rotates both query heads itself and moves them to the decode layout
    // through its own LDS rows (no workgroup barrier); the last wave of the last piece also
    // quantizes the new K and V rows (rk1.. below) for the cache and for its own use.
    uint16_t rq1[2], rq2[2], rqw1 = 0, rqw2 = 0, rcs = 0, rsn = 0;
    uint16_t rk1 = 0, rk2 = 0, rkw1 = 0, rkw2 = 0, rv1 = 0, rv2 = 0;
    float rc1 = 0.f, rc2 = 0.f;
    // the new K/V row is written to the cache by the first pair's workgroup only (the others
    // compute it for their own use)
    const bool kv_wave = last && wave == WAVES - 1;
    const bool kv_write = kv_wave && pair == 0;
    if constexpr (ROPE) {
        const float* cal =
            a.c.k_calibration + slot * a.c.cal_stride_slot + hk * a.c.cal_stride_head;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint16_t* src = a.q + b * a.q_sb + (h ? qh1 : qh0) * a.q_sh;
            rq1[h] = src[lane];
            rq2[h] = src[lane + 64];
        }
        rqw1 = a.q_norm[lane];
        rqw2 = a.q_norm[lane + 64];
        rcs = a.cos[b * a.cos_sb + lane];
        rsn = a.sin[b * a.sin_sb + lane];
        rc1 = cal[lane];
        rc2 = cal[lane + 64];
        if (kv_wave) {
            const uint16_t* kp = a.k_new + b * a.k_sb + hk * a.k_sh;
            const uint16_t* vp = a.v_new + b * a.v_sb + hk * a.v_sh;
            rk1 = kp[lane];
            rk2 = kp[lane + 64];
            rkw1 = a.k_norm[lane];
            rkw2 = a.k_norm[lane + 64];
            rv1 = vp[lane];
            rv2 = vp[lane + 64];
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint16_t* qp = a.q + b * a.q_sb + (h ? qh1 : qh0) * a.q_sh + 16 * cc;
            qraw[h][0] = *reinterpret_cast<const uint4*>(qp);
            qraw[h][1] = *reinterpret_cast<const uint4*>(qp + 8);
        }
    }
    // The first K/V block is requested with q, in the same memory round trip; the scheduling
    // barrier keeps the compiler from sinking the requests below q's conversion.
    int t0 = t_begin + wave * DA_TOK_WAVE;
    KVRegs kr, vr;
    load_block(kr, rk, rks, t0 + 4 * g, cc);
    load_block(vr, rv, rvs, t0 + 4 * g, cc);
    __builtin_amdgcn_sched_barrier(0);
    __shared__ __attribute__((aligned(16))) uint16_t s_q[ROPE ? WAVES : 1][2][DA_D];
    __shared__ __attribute__((aligned(16))) int8_t s_new[2][DA_D];
    __shared__ float s_new_scale[2];
    if constexpr (ROPE) {
        // fused_rope_kv_decode's arithmetic (the same device functions): RMSNorm and RoPE, q
        // times the calibration rounded to bf16, K divided by the calibration, K and V
        // quantized; the new row goes to the cache at column n_end - 1 and, with its scales,
        // to LDS for the last wave's own use
        const float cs = bf16_to_f32(rcs), sn = bf16_to_f32(rsn);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float o1, o2;
            norm_rope_row(bf16_to_f32(rq1[h]), bf16_to_f32(rq2[h]), bf16_to_f32(rqw1),
                          bf16_to_f32(rqw2), cs, sn, a.eps, o1, o2);
            s_q[wave][h][lane] = (uint16_t)f32_to_bf16_rne(o1 * rc1);
            s_q[wave][h][lane + 64] = (uint16_t)f32_to_bf16_rne(o2 * rc2);
        }
        if (kv_wave) {
            const int64_t col = n_end - 1;
            const int64_t base =
                slot * a.c.stride_slot + hk * a.c.stride_head + col * a.c.stride_tok;
            const int64_t sidx = slot * a.c.scale_stride_slot + hk * a.c.scale_stride_head + col;
            float o1, o2;
            norm_rope_row(bf16_to_f32(rk1), bf16_to_f32(rk2), bf16_to_f32(rkw1),
                          bf16_to_f32(rkw2), cs, sn, a.eps, o1, o2);
            int32_t q1, q2;
            const float sk = quantize_row_wave(o1 / rc1, o2 / rc2, q1, q2);
            if (kv_write) {
                a.c.k[base + lane] = (int8_t)q1;
                a.c.k[base + lane + 64] = (int8_t)q2;
            }
            s_new[0][lane] = (int8_t)q1;
            s_new[0][lane + 64] = (int8_t)q2;
            const float sv = quantize_row_wave(bf16_to_f32(rv1), bf16_to_f32(rv2), q1, q2);
            if (kv_write) {
                a.c.v[base + lane] = (int8_t)q1;
                a.c.v[base + lane + 64] = (int8_t)q2;
            }
            s_new[1][lane] = (int8_t)q1;
            s_new[1][lane + 64] = (int8_t)q2;
            if (lane == 0) {
                if (kv_write) {
                    a.c.k_scale[sidx] = sk;
                    a.c.v_scale[sidx] = sv;
                }
                s_new_scale[0] = sk;
                s_new_scale[1] = sv;
            }
        }
        // the wave's own LDS rows: its writes are visible to its later reads once the LDS
        // operations are ordered within the wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            qraw[h][0] = *reinterpret_cast<const uint4*>(&s_q[wave][h][16 * cc]);
            qraw[h][1] = *reinterpret_cast<const uint4*>(&s_q[wave][h][16 * cc + 8]);
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 u0 = qraw[h][0], u1 = qraw[h][1];
        const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
        float f[16];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            f[2 * i] = bf16lo(w[i]);
            f[2 * i + 1] = bf16hi(w[i]);
            amax = fmaxf(amax, fmaxf(fabsf(f[2 * i]), fabsf(f[2 * i + 1])));
        }
        amax = fmaxf(amax, dpp<DPP_XOR1>(amax));
        amax = fmaxf(amax, dpp<DPP_XOR2>(amax));
        amax = fmaxf(amax, dpp<DPP_HALF_MIRROR>(amax));
        int e = 0;
        frexpf(amax, &e);
        const float sc = amax > 0.0f ? ldexpf(1.0f, 14 - e) : 1.0f;  // amax*sc in [2^13, 2^14)
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const _Float16 lo = (_Float16)(f[2 * i] * sc), hi = (_Float16)(f[2 * i + 1] * sc);
            qh[h][i] = half2_t{lo, hi};
            s += (float)lo + (float)hi;
        }
        qoff[h] = __int_as_float(uniform(__float_as_int(sum8(s) * (-OFFSET / 8.0f))));
        kmul[h] = __int_as_float(uniform(__float_as_int(a.scale_log2 / sc)));
    }

    LaneState st;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        st.m[h] = -INFINITY;
        st.l[h] = 0.0f;
        st.ps[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) st.acc[h][j] = 0.0f;
    }
    st.ve = 0.0f;
    st.vlo = (uint32_t)(8 + 127) << 23;

    // Rolling pipeline: the next block's K is requested as soon as this block's scores are
    // done and its V as soon as this block's PV is done, so every load has half a block of
    // VALU work to hide behind without extra registers. Requests past the piece's end fall
    // outside the buffer range and return zeros without touching memory.
    // this wave's blocks: w, w + 8, ... of the piece's 32-token blocks, counted up front
    const int nb = (t_end - t_begin + DA_TOK_WAVE - 1) / DA_TOK_WAVE;
    const int cw = wave < nb ? (nb - wave + WAVES - 1) / WAVES : 0;
    int nfull = cw;
    if (cw > 0 && t_begin + DA_TOK_WAVE * (wave + WAVES * (cw - 1)) + DA_TOK_WAVE > t_end)
        --nfull;  // the piece's last, partial block
    float s[DA_U][2];
    for (int j = 0; j < nfull; ++j, t0 += TOK_WG) {
        block_scores<false>(s, kr, qh, qoff, t0 + 4 * g, t_end);
        load_block(kr, rk, rks, t0 + TOK_WG + 4 * g, cc);
        block_pv(st, s, vr, kmul);
        load_block(vr, rv, rvs, t0 + TOK_WG + 4 * g, cc);
    }
    // the lane group derived afresh from the thread index for the masked blocks below: kept
    // from the prologue it is a register the loop needs
    int tid_m = lane_id();
    asm volatile("" : "+v"(tid_m));
    tid_m += IE_WAVE * wave;
    const int gm = (tid_m & 63) >> 3;
    if (nfull < cw) {
        block_scores<true>(s, kr, qh, qoff, t0 + 4 * gm, t_end);
        block_pv(st, s, vr, kmul);
    }
    if (ROPE && kv_wave) {
        // the new token, as a block whose other tokens are masked: lane group 0 holds its row
        KVRegs kn, vn;
#pragma unroll
        for (int u = 0; u < DA_U; ++u) kn.x[u] = vn.x[u] = v4u{0u, 0u, 0u, 0u};
        kn.scale = vn.scale = v4u{0u, 0u, 0u, 0u};
        if (gm == 0) {
            const int cm = tid_m & 7;
            kn.x[0] = *reinterpret_cast<const v4u*>(&s_new[0][16 * cm]);
            vn.x[0] = *reinterpret_cast<const v4u*>(&s_new[1][16 * cm]);
            kn.scale[0] = __float_as_uint(s_new_scale[0]);
            vn.scale[0] = __float_as_uint(s_new_scale[1]);
        }
        block_scores<true>(s, kn, qh, qoff, n_end - 1 + 4 * gm, n_end);
        block_pv(st, s, vn, kmul);
    }

    float (&m)[2] = st.m;
    float (&l)[2] = st.l;
    float (&ps)[2] = st.ps;
    float (&acc)[2][16] = st.acc;

    // ---- merge the 8 lane groups of the wave ----
    float mw[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float mx = m[h];
        mx = fmaxf(mx, dpp<DPP_ROR8>(mx));
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        mw[h] = mx;
        const float f = m[h] == -INFINITY ? 0.0f : exp2_safe(m[h] - mx);
        float lf = l[h] * f;
        lf += dpp<DPP_ROR8>(lf);
        lf += shfl_xor(lf, 16);
        lf += shfl_xor(lf, 32);
        l[h] = lf;
        const float off = ps[h] * OFFSET;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            float x = (acc[h][j] - off) * f;
            x += dpp<DPP_ROR8>(x);
            x += shfl_xor(x, 16);
            x += shfl_xor(x, 32);
            acc[h][j] = x;
        }
    }

    // ---- merge the waves through LDS ----
    __shared__ float s_acc[WAVES][2][DA_D];
    __shared__ float s_m[WAVES][2], s_l[WAVES][2];
    // the lane's channel group, derived afresh from the thread index: keeping the prologue's copy
    // alive across the loop costs a register the loop needs
    int tid = lane_id();
    asm volatile("" : "+v"(tid));
    tid += IE_WAVE * wave;
    const int ccm = tid & 7;
    if (g == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int j = 0; j < 16; ++j) s_acc[wave][h][16 * ccm + j] = acc[h][j];
            if (ccm == 0) {
                s_m[wave][h] = mw[h];
                s_l[wave][h] = l[h];
            }
        }
    }
    __syncthreads();
    // one (query head, channel) output per thread, or two with 2-wave workgroups; threads past
    // the 256 outputs stay for the barriers
    constexpr int PER = (2 * DA_D + THREADS - 1) / THREADS;
    float num[PER], den[PER], mxo[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int idx = tid + u * THREADS;
        const int h = (idx >> 7) & 1, d = idx & 127;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) mx = fmaxf(mx, s_m[w][h]);
        num[u] = 0.0f;
        den[u] = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float mwv = s_m[w][h];
            const float f = mwv == -INFINITY ? 0.0f : exp2_safe(mwv - mx);
            num[u] += s_acc[w][h][d] * f;
            den[u] += s_l[w][h] * f;
        }
        mxo[u] = mx;
    }
    auto out_of = [&](int u) {
        const int idx = tid + u * THREADS;
        return a.out + b * a.o_sb + (qh0 + ((idx >> 7) & 1)) * a.o_sh + (idx & 127);
    };
    // thread idx's output exists (the second head of a one-head pair does not)
    auto active = [&](int u) {
        const int idx = tid + u * THREADS;
        return idx < (has2 ? 2 : 1) * DA_D;
    };
    if (wk.needed == 1) {
#pragma unroll
        for (int u = 0; u < PER; ++u)
            if (active(u)) *out_of(u) = (uint16_t)f32_to_bf16_rne(num[u] / den[u]);
        return;
    }
    // A sequence of several pieces: each piece publishes its partial (the sequence's pieces
    // are consecutive work entries) and counts itself in; the piece that arrives last merges
    // them all (kernels.py:216-264, in base 2, pieces in order) and resets the count for the
    // next call. The partials are written and read with device-coherent accesses.
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        if (!active(u)) continue;
        const int idx = tid + u * THREADS;
        const int d = idx & 127;
        const int64_t row = (int64_t)(qh0 + ((idx >> 7) & 1)) * a.nwork + item;
        st_dev(a.part_acc + row * DA_D + d, num[u]);
        if (d == 0) {
            st_dev(a.part_m + row, mxo[u]);
            st_dev(a.part_l + row, den[u]);
        }
    }
    if (!arrive_last(a.arrivals + b * a.units + unit, wk.needed)) return;
    const int needed = wk.needed;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        if (!active(u)) continue;
        const int idx = tid + u * THREADS;
        const int d = idx & 127;
        const int64_t row0 = (int64_t)(qh0 + ((idx >> 7) & 1)) * a.nwork + (item - split);
        constexpr int CB = 8;  // partials per load batch: one memory round trip each
        float av[CB], ml[CB][2];
        auto load_batch = [&](int s0) {
#pragma unroll
            for (int v = 0; v < CB; ++v) {
                const bool in = s0 + v < needed;
                av[v] = in ? ld_dev(a.part_acc + (row0 + s0 + v) * DA_D + d) : 0.0f;
                ml[v][0] = in ? ld_dev(a.part_m + row0 + s0 + v) : -INFINITY;
                ml[v][1] = in ? ld_dev(a.part_l + row0 + s0 + v) : 0.0f;
            }
        };
        // the largest partial maximum; with at most CB pieces the batch loaded here is the
        // only one the merge needs
        load_batch(0);
        float pm = -INFINITY;
#pragma unroll
        for (int v = 0; v < CB; ++v) pm = fmaxf(pm, ml[v][0]);
        for (int s0 = CB; s0 < needed; s0 += CB) {
            float mv[CB];
#pragma unroll
            for (int v = 0; v < CB; ++v)
                mv[v] = s0 + v < needed ? ld_dev(a.part_m + row0 + s0 + v) : -INFINITY;
#pragma unroll
            for (int v = 0; v < CB; ++v) pm = fmaxf(pm, mv[v]);
        }
        float nm = 0.0f, dn = 0.0f;
        for (int s0 = 0; s0 < needed; s0 += CB) {
            if (s0 > 0) load_batch(s0);
#pragma unroll
            for (int v = 0; v < CB; ++v) {
                if (s0 + v < needed) {
                    const float f = ml[v][0] == -INFINITY ? 0.0f : exp2_safe(ml[v][0] - pm);
                    nm += av[v] * f;
                    dn += ml[v][1] * f;
                }
            }
        }
        *out_of(u) = (uint16_t)f32_to_bf16_rne(nm / dn);
    }
}

// grid (work entries), block 64: the decode kernel's work list, one entry per workgroup index w
// of its grid, computed by the same device code (decode_assign), written as
// rows[w] = (b, split, needed, piece).
__global__ __launch_bounds__(64) void decode_plan_kernel(const int32_t* __restrict__ cached_lens,
                                                         const int32_t* __restrict__ num_decoding,
                                                         int batch, int target,
                                                         int32_t* __restrict__ rows) {
    const int lane = threadIdx.x;
    const int raw0 = lane < batch ? cached_lens[lane] : 0;
    const int nd = num_decoding[0];
    const Work wk = decode_assign(cached_lens, nd, blockIdx.x, target, raw0);
    if (lane == 0) {
        int32_t* r = rows + 4 * blockIdx.x;
        r[0] = wk.b;
        r[1] = wk.split;
        r[2] = wk.needed;
        r[3] = wk.piece;
    }
}

// A decode step's per-step launch (ie_decode_step_prologue): the first ngather workgroups copy
// 512-element pieces of the embedding rows x[b] = embed[ids[b]] (zeros for an id outside
// [0, vocab)), one 16-byte load per lane; the next nrope ones the RoPE tables of positions
// cached_lens[0, batch) (64 entries each, rope_table_entry); the rest the work list, as
// decode_plan_kernel writes it.
__global__ __launch_bounds__(64) void decode_prologue_kernel(
    const int32_t* __restrict__ cached_lens, const int32_t* __restrict__ num_decoding, int batch,
    int target, int32_t* __restrict__ rows, const float* __restrict__ inv, int half,
    uint16_t* __restrict__ cosv, uint16_t* __restrict__ sinv, int nrope,
    const int64_t* __restrict__ ids, const uint16_t* __restrict__ embed, int64_t es,
    int64_t vocab, int dim, uint16_t* __restrict__ x, int64_t xs) {
    const int lane = threadIdx.x;
    const int pieces = (dim + 8 * IE_WAVE - 1) / (8 * IE_WAVE);
    const int ngather = batch * pieces;
    int w = blockIdx.x;
    if (w < ngather) {
        const int b = w / pieces, c = (w % pieces) * 8 * IE_WAVE + 8 * lane;
        if (c >= dim) return;  // dim a multiple of 8
        const int64_t id = ids[b];
        const bool ok = id >= 0 && id < vocab;
        const uint4 v = ok ? *reinterpret_cast<const uint4*>(embed + id * es + c)
                           : make_uint4(0u, 0u, 0u, 0u);
        *reinterpret_cast<uint4*>(x + (int64_t)b * xs + c) = v;
        return;
    }
    w -= ngather;
    if (w < nrope) {
        const int64_t i = (int64_t)w * IE_WAVE + lane;
        if (i < (int64_t)batch * half) rope_table_entry(cached_lens, inv, i, half, cosv, sinv);
        return;
    }
    w -= nrope;
    const int raw0 = lane < batch ? cached_lens[lane] : 0;
    const int nd = num_decoding[0];
    const Work wk = decode_assign(cached_lens, nd, w, target, raw0);
    if (lane == 0) {
        int32_t* r = rows + 4 * w;
        r[0] = wk.b;
        r[1] = wk.split;
        r[2] = wk.needed;
        r[3] = wk.piece;
    }
}

// Workspace: the arrival counts (one per sequence and KV head; zero on entry, and every call
// leaves them zero), then fp32 partials (acc, m, l) of every (query head, work entry): one per
// piece, since pieces never outnumber the decode launch's work entries per KV head. The count
// region has room for DA_COUNT_CAP sequences and DA_COUNT_HEADS query heads whatever the batch
// and the head count, so calls of any batch and head count up to those agree on where the
// counts are and their partials never land on them: one workspace serves them all. (Sized by
// the call's own head count, a call with fewer query heads would write partials over the count
// words of a later call with more sequences or heads.) A larger batch or head count gets a
// count region of its own size.
constexpr int DA_COUNT_CAP = 1024;
constexpr int DA_COUNT_HEADS = 128;
struct Layout {
    int waves, target, nwork;
    size_t arr_off, acc_off, m_off, l_off, bytes;
};

// The layout of a launch of `units` units (decode_units). The count region has a count per
// sequence and query head, the most any GQA ratio needs (one per sequence and unit), so every
// launch of a batch size finds its counts and partials at the same offsets; the partial rows
// (one per query head and work entry) fit the largest grid any ratio launches, that of
// cdiv(hq, 2) units (workspace_size_layout).
static Layout workspace_layout(int batch, int hq, int units) {
    Layout L;
    batch = std::max(batch, 0);
    L.waves = decode_waves(batch, units);
    L.target = decode_target(units, L.waves);
    L.nwork = batch <= L.target ? L.target : L.target + batch;
    const size_t rows = (size_t)hq * L.nwork;
    L.arr_off = 0;
    L.acc_off = ((size_t)std::max(batch, DA_COUNT_CAP) * std::max(hq, DA_COUNT_HEADS) *
                     sizeof(uint32_t) + 255) / 256 * 256;
    L.m_off = L.acc_off + rows * DA_D * sizeof(float);
    L.l_off = L.m_off + rows * sizeof(float);
    L.bytes = L.l_off + rows * sizeof(float);
    return L;
}
static Layout workspace_size_layout(int batch, int hq) {
    return workspace_layout(batch, hq, std::max(1, (hq + 1) / 2));
}

}  // namespace ie

using namespace ie;

extern "C" size_t ie_decode_attention_workspace_counts_bytes(int32_t batch,
                                                             int32_t num_q_heads) {
    if (num_q_heads <= 0) return 0;
    return workspace_size_layout(batch, num_q_heads).acc_off;
}

extern "C" int32_t ie_decode_attention_max_splits(int32_t num_units) {
    return decode_target(num_units, 2);  // the largest target of any launch shape
}

extern "C" int32_t ie_decode_attention_target(int32_t batch, int32_t num_units) {
    if (batch <= 0 || num_units <= 0) return 0;
    return decode_target(num_units, decode_waves(batch, num_units));
}

extern "C" size_t ie_decode_attention_workspace_size(int32_t batch, int32_t num_q_heads,
                                                     int32_t head_dim) {
    (void)head_dim;
    if (num_q_heads <= 0) return 0;
    return workspace_size_layout(batch, num_q_heads).bytes;
}

// q_rows16: q is read in 16-byte pieces (the plain form; the fused form reads q two bytes per
// lane, as fused_rope_kv_decode does).
static hipError_t check_decode(const ie_bf16* q, int32_t batch, int32_t num_q_heads,
                               const ie_kv_cache* cache, const int32_t* cached_lens,
                               const int32_t* slot_ids, const int32_t* num_decoding,
                               const ie_bf16* out, int64_t q_sb, int64_t q_sh, void* workspace,
                               size_t workspace_bytes, Layout* L, bool q_rows16 = true) {
    hipError_t e = check_cache(cache);
    if (e != hipSuccess) return e;
    IE_REQUIRE(batch >= 0, "negative batch");
    IE_REQUIRE(num_q_heads > 0 && num_q_heads % cache->num_kv_heads == 0 &&
                   num_q_heads / cache->num_kv_heads <= 16,
               "num_q_heads must be num_kv_heads times a GQA ratio of 1 to 16");
    if (batch == 0) return hipSuccess;
    IE_REQUIRE(q && cached_lens && slot_ids && num_decoding && out, "null pointer");
    IE_REQUIRE(!q_rows16 ||
                   ((reinterpret_cast<uintptr_t>(q) & 15) == 0 && q_sb % 8 == 0 && q_sh % 8 == 0),
               "q rows must be 16-byte aligned with contiguous head_dim");
    *L = workspace_layout(batch, num_q_heads,
                          decode_units(num_q_heads, (int)cache->num_kv_heads));
    IE_REQUIRE(workspace != nullptr && workspace_bytes >= L->bytes, "workspace too small");
    IE_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0, "workspace must be aligned");
    return hipSuccess;
}

// The arguments both forms share; the fused form's own fields stay null.
static DecodeArgs decode_args(const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h,
                              int32_t batch, int32_t num_q_heads, const ie_kv_cache* cache,
                              const int32_t* cached_lens, const int32_t* slot_ids,
                              const int32_t* num_decoding, float scale, ie_bf16* out,
                              int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                              const Layout& L) {
    DecodeArgs a{};
    a.q = (const uint16_t*)q;
    a.q_sb = q_stride_b;
    a.q_sh = q_stride_h;
    a.c = *cache;
    a.cached_lens = cached_lens;
    a.slot_ids = slot_ids;
    a.num_decoding = num_decoding;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.out = (uint16_t*)out;
    a.o_sb = out_stride_b;
    a.o_sh = out_stride_h;
    char* ws = (char*)workspace;
    a.part_acc = (float*)(ws + L.acc_off);
    a.part_m = (float*)(ws + L.m_off);
    a.part_l = (float*)(ws + L.l_off);
    a.arrivals = (uint32_t*)(ws + L.arr_off);
    a.target = L.target;
    a.nwork = L.nwork;
    a.hq = num_q_heads;
    a.hkv = (int)cache->num_kv_heads;
    a.ratio = num_q_heads / a.hkv;
    a.npairs = (a.ratio + 1) / 2;
    a.units = a.hkv * a.npairs;
    a.batch = batch;
    return a;
}

template <bool ROPE>
static hipError_t decode_launch(DecodeArgs& a, const Layout& L, int32_t batch,
                                const ie_kv_cache* cache, hipStream_t stream) {
    // pieces number at most target + nd, and at most target when nd <= target (decode_piece):
    // with batch <= target the grid needs no spare workgroups, which would otherwise hold
    // resident slots while they find out that they are idle
    const unsigned pieces = (unsigned)L.nwork;
    // The order in which the dispatcher hands out workgroups (same results either way): the KV
    // heads of one piece side by side measured 9 % faster at B=64 ctx=1024, but 0.4-0.8 %
    // slower at B=64 ctx=4096 and 3-4 % slower at config 5 (B=32); the host cannot tell the
    // context lengths apart, so the pieces of one head go side by side unless
    // IE_DECODE_HEAD_FAST_MIN_BATCH (0: never) is set.
    a.head_fast = IE_DECODE_HEAD_FAST_MIN_BATCH > 0 && batch >= IE_DECODE_HEAD_FAST_MIN_BATCH &&
                  pieces <= 65535;  // the grid's y dimension holds at most 65535
    const dim3 grid = a.head_fast ? dim3((unsigned)a.hkv, pieces, (unsigned)a.npairs)
                                  : dim3(pieces, (unsigned)a.hkv, (unsigned)a.npairs);
    if (a.ratio == 2) {
        switch (L.waves) {
            case 8: hipLaunchKernelGGL((decode_attention_kernel<8, ROPE, true>), grid, dim3(512), 0, stream, a); break;
            case 4: hipLaunchKernelGGL((decode_attention_kernel<4, ROPE, true>), grid, dim3(256), 0, stream, a); break;
            default: hipLaunchKernelGGL((decode_attention_kernel<2, ROPE, true>), grid, dim3(128), 0, stream, a); break;
        }
    } else {
        switch (L.waves) {
            case 8: hipLaunchKernelGGL((decode_attention_kernel<8, ROPE, false>), grid, dim3(512), 0, stream, a); break;
            case 4: hipLaunchKernelGGL((decode_attention_kernel<4, ROPE, false>), grid, dim3(256), 0, stream, a); break;
            default: hipLaunchKernelGGL((decode_attention_kernel<2, ROPE, false>), grid, dim3(128), 0, stream, a); break;
        }
    }
    return hipGetLastError();
}

// A precomputed work list must cover the launch's grid (plan_rows >= its work entries).
static hipError_t check_plan(const int32_t* plan, int64_t plan_rows, const Layout& L) {
    IE_REQUIRE(plan != nullptr, "null plan");
    IE_REQUIRE(plan_rows >= L.nwork,
               "plan must hold ie_decode_attention_grid(batch, units) rows");
    IE_REQUIRE((reinterpret_cast<uintptr_t>(plan) & 15) == 0, "plan must be 16-byte aligned");
    return hipSuccess;
}

static hipError_t decode_plain(const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h,
                               int32_t batch, int32_t num_q_heads, const ie_kv_cache* cache,
                               const int32_t* cached_lens, const int32_t* slot_ids,
                               const int32_t* num_decoding, float scale, ie_bf16* out,
                               int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                               size_t workspace_bytes, const int32_t* plan, int64_t plan_rows,
                               bool planned, hipStream_t stream) {
    Layout L{};
    hipError_t e = check_decode(q, batch, num_q_heads, cache, cached_lens, slot_ids, num_decoding,
                                out, q_stride_b, q_stride_h, workspace, workspace_bytes, &L);
    if (e != hipSuccess || batch == 0) return e;
    if (planned && (e = check_plan(plan, plan_rows, L)) != hipSuccess) return e;
    DecodeArgs a = decode_args(q, q_stride_b, q_stride_h, batch, num_q_heads, cache, cached_lens,
                               slot_ids, num_decoding, scale, out, out_stride_b, out_stride_h,
                               workspace, L);
    a.plan = planned ? plan : nullptr;
    return decode_launch<false>(a, L, batch, cache, stream);
}

extern "C" hipError_t ie_decode_attention(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, int32_t batch, int32_t num_q_heads,
    const ie_kv_cache* cache, const int32_t* cached_lens, const int32_t* slot_ids,
    const int32_t* num_decoding, float scale, ie_bf16* out, int64_t out_stride_b,
    int64_t out_stride_h, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return decode_plain(q, q_stride_b, q_stride_h, batch, num_q_heads, cache, cached_lens,
                        slot_ids, num_decoding, scale, out, out_stride_b, out_stride_h, workspace,
                        workspace_bytes, nullptr, 0, false, stream);
}

extern "C" hipError_t ie_decode_attention_planned(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, int32_t batch, int32_t num_q_heads,
    const ie_kv_cache* cache, const int32_t* cached_lens, const int32_t* slot_ids,
    const int32_t* num_decoding, const int32_t* plan, int64_t plan_rows, float scale,
    ie_bf16* out, int64_t out_stride_b, int64_t out_stride_h, void* workspace,
    size_t workspace_bytes, hipStream_t stream) {
    return decode_plain(q, q_stride_b, q_stride_h, batch, num_q_heads, cache, cached_lens,
                        slot_ids, num_decoding, scale, out, out_stride_b, out_stride_h, workspace,
                        workspace_bytes, plan, plan_rows, true, stream);
}

static hipError_t decode_rope(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, const ie_bf16* k,
    int64_t k_stride_b, int64_t k_stride_h, const ie_bf16* v, int64_t v_stride_b,
    int64_t v_stride_h, const ie_bf16* q_norm_weight, const ie_bf16* k_norm_weight,
    const ie_bf16* cos, int64_t cos_stride_b, const ie_bf16* sin, int64_t sin_stride_b,
    float eps, int32_t batch, int32_t num_q_heads, const ie_kv_cache* cache,
    const int32_t* cached_lens, const int32_t* slot_ids, const int32_t* num_decoding,
    const int32_t* plan, int64_t plan_rows, bool planned, float scale, ie_bf16* out,
    int64_t out_stride_b, int64_t out_stride_h, void* workspace, size_t workspace_bytes,
    hipStream_t stream) {
    Layout L{};
    hipError_t e = check_decode(q, batch, num_q_heads, cache, cached_lens, slot_ids, num_decoding,
                                out, q_stride_b, q_stride_h, workspace, workspace_bytes, &L,
                                false);
    if (e != hipSuccess || batch == 0) return e;
    IE_REQUIRE(k && v && q_norm_weight && k_norm_weight && cos && sin, "null pointer");
    if (planned && (e = check_plan(plan, plan_rows, L)) != hipSuccess) return e;
    DecodeArgs a = decode_args(q, q_stride_b, q_stride_h, batch, num_q_heads, cache, cached_lens,
                               slot_ids, num_decoding, scale, out, out_stride_b, out_stride_h,
                               workspace, L);
    a.plan = planned ? plan : nullptr;
    a.k_new = (const uint16_t*)k;
    a.k_sb = k_stride_b;
    a.k_sh = k_stride_h;
    a.v_new = (const uint16_t*)v;
    a.v_sb = v_stride_b;
    a.v_sh = v_stride_h;
    a.q_norm = (const uint16_t*)q_norm_weight;
    a.k_norm = (const uint16_t*)k_norm_weight;
    a.cos = (const uint16_t*)cos;
    a.sin = (const uint16_t*)sin;
    a.cos_sb = cos_stride_b;
    a.sin_sb = sin_stride_b;
    a.eps = eps;
    return decode_launch<true>(a, L, batch, cache, stream);
}

extern "C" hipError_t ie_decode_attention_rope(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, const ie_bf16* k,
    int64_t k_stride_b, int64_t k_stride_h, const ie_bf16* v, int64_t v_stride_b,
    int64_t v_stride_h, const ie_bf16* q_norm_weight, const ie_bf16* k_norm_weight,
    const ie_bf16* cos, int64_t cos_stride_b, const ie_bf16* sin, int64_t sin_stride_b,
    float eps, int32_t batch, int32_t num_q_heads, const ie_kv_cache* cache,
    const int32_t* cached_lens, const int32_t* slot_ids, const int32_t* num_decoding,
    float scale, ie_bf16* out, int64_t out_stride_b, int64_t out_stride_h, void* workspace,
    size_t workspace_bytes, hipStream_t stream) {
    return decode_rope(q, q_stride_b, q_stride_h, k, k_stride_b, k_stride_h, v, v_stride_b,
                       v_stride_h, q_norm_weight, k_norm_weight, cos, cos_stride_b, sin,
                       sin_stride_b, eps, batch, num_q_heads, cache, cached_lens, slot_ids,
                       num_decoding, nullptr, 0, false, scale, out, out_stride_b, out_stride_h,
                       workspace, workspace_bytes, stream);
}

extern "C" hipError_t ie_decode_attention_rope_planned(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, const ie_bf16* k,
    int64_t k_stride_b, int64_t k_stride_h, const ie_bf16* v, int64_t v_stride_b,
    int64_t v_stride_h, const ie_bf16* q_norm_weight, const ie_bf16* k_norm_weight,
    const ie_bf16* cos, int64_t cos_stride_b, const ie_bf16* sin, int64_t sin_stride_b,
    float eps, int32_t batch, int32_t num_q_heads, const ie_kv_cache* cache,
    const int32_t* cached_lens, const int32_t* slot_ids, const int32_t* num_decoding,
    const int32_t* plan, int64_t plan_rows, float scale, ie_bf16* out, int64_t out_stride_b,
    int64_t out_stride_h, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return decode_rope(q, q_stride_b, q_stride_h, k, k_stride_b, k_stride_h, v, v_stride_b,
                       v_stride_h, q_norm_weight, k_norm_weight, cos, cos_stride_b, sin,
                       sin_stride_b, eps, batch, num_q_heads, cache, cached_lens, slot_ids,
                       num_decoding, plan, plan_rows, true, scale, out, out_stride_b,
                       out_stride_h, workspace, workspace_bytes, stream);
}

extern "C" int32_t ie_decode_attention_grid(int32_t batch, int32_t num_units) {
    if (batch <= 0 || num_units <= 0) return 0;
    const int target = ie_decode_attention_target(batch, num_units);
    return batch <= target ? target : target + batch;
}

extern "C" hipError_t ie_decode_step_prologue(
    const int32_t* cached_lens, const int32_t* num_decoding, int32_t batch, int32_t num_units,
    int32_t* rows, const float* inv_freq, int32_t half_dim, ie_bf16* cos_out, ie_bf16* sin_out,
    const int64_t* ids, const ie_bf16* embed, int64_t embed_stride, int64_t vocab,
    int32_t model_dim, ie_bf16* x, int64_t x_stride, hipStream_t stream) {
    IE_REQUIRE(batch >= 0 && num_units > 0 && half_dim > 0 && vocab > 0 && model_dim > 0,
               "bad sizes");
    if (batch == 0) return hipSuccess;
    IE_REQUIRE(cached_lens && num_decoding && rows && inv_freq && cos_out && sin_out && ids &&
                   embed && x,
               "null pointer");
    IE_REQUIRE(model_dim % 8 == 0 && embed_stride % 8 == 0 && x_stride % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(embed) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(x) & 15) == 0,
               "embedding and x rows must be 16-byte aligned, model_dim a multiple of 8");
    const int target = ie_decode_attention_target(batch, num_units);
    const int nplan = ie_decode_attention_grid(batch, num_units);
    const int64_t nrope = ((int64_t)batch * half_dim + IE_WAVE - 1) / IE_WAVE;
    const int64_t ngather = (int64_t)batch * ((model_dim + 8 * IE_WAVE - 1) / (8 * IE_WAVE));
    IE_REQUIRE(nplan + nrope + ngather < (1LL << 31), "too many workgroups");
    hipLaunchKernelGGL(decode_prologue_kernel, dim3((unsigned)(ngather + nrope + nplan)),
                       dim3(IE_WAVE), 0, stream, cached_lens, num_decoding, batch, target,
                       rows, inv_freq, (int)half_dim, (uint16_t*)cos_out, (uint16_t*)sin_out,
                       (int)nrope, ids, (const uint16_t*)embed, embed_stride, vocab,
                       (int)model_dim, (uint16_t*)x, x_stride);
    return hipGetLastError();
}

extern "C" hipError_t ie_decode_attention_plan(const int32_t* cached_lens,
                                               const int32_t* num_decoding, int32_t batch,
                                               int32_t num_units, int32_t* rows,
                                               hipStream_t stream) {
    IE_REQUIRE(batch >= 0 && num_units > 0, "bad sizes");
    if (batch == 0) return hipSuccess;
    IE_REQUIRE(cached_lens && num_decoding && rows, "null pointer");
    const int target = ie_decode_attention_target(batch, num_units);
    hipLaunchKernelGGL(decode_plan_kernel, dim3((unsigned)ie_decode_attention_grid(batch, num_units)),
                       dim3(IE_WAVE), 0, stream, cached_lens, num_decoding, batch, target, rows);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// The entry point that allocates nothing: ie_decode_attention with its workspace in a static
// device array of DA_SCRATCH_BYTES, which every device the library runs on holds until the
// process ends (16 MiB: the arrival counts and partials of up to 1,024 sequences, the batches
// that share one count region). The array's name is only a host-side stand-in for the device copy, so
// its address on each device is looked up once, with that device current, and only that
// address is passed to the kernels. The array starts zeroed, as the workspace contract asks,
// and every call leaves the arrival counts zeroed again. All calls on one device share the array,
// so calls that overlap on one device (different streams, or threads without ordering) race.
// ---------------------------------------------------------------------------------------------
namespace {
constexpr size_t DA_SCRATCH_BYTES = size_t(16) << 20;
constexpr int DA_SCRATCH_DEVICES = 64;
__device__ __align__(256) unsigned char scratch[DA_SCRATCH_BYTES];
std::mutex scratch_mu;
void* scratch_ptr[DA_SCRATCH_DEVICES];

// This device's copy of `scratch` (resolved on the first call made with the device current).
hipError_t scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    IE_REQUIRE(dev >= 0 && dev < DA_SCRATCH_DEVICES, "device index out of range");
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        IE_REQUIRE(p != nullptr, "no device address for the decode scratch");
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return hipSuccess;
}
}  // namespace

extern "C" size_t ie_decode_attention_noalloc_max_bytes(void) { return DA_SCRATCH_BYTES; }

extern "C" hipError_t ie_decode_attention_noalloc(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, int32_t batch, int32_t num_q_heads,
    const ie_kv_cache* cache, const int32_t* cached_lens, const int32_t* slot_ids,
    const int32_t* num_decoding, float scale, ie_bf16* out, int64_t out_stride_b,
    int64_t out_stride_h, hipStream_t stream) {
    hipError_t e = check_cache(cache);
    if (e != hipSuccess) return e;
    IE_REQUIRE(batch >= 0, "negative batch");
    if (batch == 0) return hipSuccess;
    IE_REQUIRE(num_q_heads > 0 && num_q_heads % cache->num_kv_heads == 0 &&
                   num_q_heads / cache->num_kv_heads <= 16,
               "num_q_heads must be num_kv_heads times a GQA ratio of 1 to 16");
    const Layout L =
        workspace_layout(batch, num_q_heads, decode_units(num_q_heads, (int)cache->num_kv_heads));
    IE_REQUIRE(batch <= DA_COUNT_CAP && num_q_heads <= DA_COUNT_HEADS &&
                   L.bytes <= DA_SCRATCH_BYTES,
               "batch too large for the no-alloc decode scratch (at most 1024 sequences and "
               "128 query heads in 16 MiB; use ie_decode_attention with a workspace)");
    void* ws = nullptr;
    e = scratch_address(&ws);
    if (e != hipSuccess) return e;
    return ie_decode_attention(q, q_stride_b, q_stride_h, batch, num_q_heads, cache, cached_lens,
                               slot_ids, num_decoding, scale, out, out_stride_b, out_stride_h, ws,
                               DA_SCRATCH_BYTES, stream);
}
