// Causal chunked-prefill attention over the int8 cache prefix, bf16 MFMA (gfx950).
//
// Semantics (qwen3-1.7b/kernels.py:987-1126 fed by dequantize_kv_prefix, kernels.py:868-932):
// packed row m of entry e attends to e's cached prefix — cache row slot_ids[e], columns
// [0, P), P = cu_cached[e+1] - cu_cached[e], k = q_int8 * k_scale * cal, v = q_int8 * v_scale —
// and to its own chunk rows [cu_seqlens[e], m] (bf16 k, v as given). Scores are
// dot(q, k) * D^-0.5 * log2(e); softmax in base 2; P is rounded to bf16 before PV;
// out = acc / l (as acc * (1 / l)), or 0 when l == 0.
//
// Prefix K with its scales folded out of the tile: int8 -> bf16 is exact, so the staged K tiles
// hold the raw integers and the scales go where they cost nothing extra:
//   S(row, key) = (sum_d bf16(q[d] * cal[d]) * k_int8[key][d]) * (k_scale[key] * D^-0.5 log2 e)
// (the reference rounds bf16((k_int8 * k_scale) * cal) instead: same quantity, the rounding in
// another place, well inside bf16 attention tolerance). Prefix V is staged dequantized,
// bf16(v_int8 * v_scale), exactly as the reference rounds it.
//
// Work: sub-blocks of up to PF_BM (128) packed rows of one tile of `block_m` rows (tile_start,
// -1 = no work), one query-head pair of one KV head (a unit) per workgroup. Every workgroup reads
// the tile metadata (one wave, a few hundred sub-blocks at most) and derives the same work list:
// the key range of a (sub-block, unit) pair (prefix tiles, then chunk tiles up to its last row)
// is one piece, or, when longer than T 64-key tiles, prefix pieces and chunk pieces of at most T
// tiles (or even consecutive ranges that may straddle the two), T the smallest size whose pieces
// fit one resident wave of workgroups (one per CU). Workgroup w runs piece w of the list
// (largest sub-blocks first). Unsplit pieces write `out`; split pieces
// write a bf16 partial O (normalized) and fp32 (m, l) to their slot and count themselves in,
// and the piece of a (sub-block, kv head) that arrives last merges them all (log-sum-exp) into
// `out` in the same launch. The work list can also be computed once (prefill_plan_kernel, 16
// int32 per workgroup) and handed to the launch, whose workgroups then read their row instead.
//
// Per 64-key tile: the workgroup stages K as [key][d] and V transposed as [d][key] in LDS, and
// the tile's score scales; wave w (the unit's query head w & 1, rows 32 (w >> 1)..+32) computes
//   S^T (64 keys x 32 rows) = K . Q^T   v_mfma_f32_16x16x32_bf16, A = K from LDS, B = Q^T in VGPRs
//   online softmax on S^T (a lane holds one row's scores for 16 keys)
//   O^T (128 d x 32 rows) += V^T . P^T  A = V^T from LDS, B = P^T straight from the S^T
//                                       accumulators (same key permutation in A and B)
//   l += ones . P^T                     the row sums, on the MFMA as well
// software-pipelined: the QK^T of tile j+1 beside the softmax of tile j, the PV of tile j beside
// the staging of the next K and V tiles, whose global loads were issued a step earlier.
#include <cstdlib>

#include "ie_common.h"

namespace ie {

// Phase stamps (diagnostic build only, -DIE_PREFILL_PHASE_STAMPS; the product build compiles
// them out): thread 0 of workgroup w < PF_STAMP_WGS records the 100 MHz real-time clock at
//   0 start, 1 work list known, 2 first tile's scores done, 3 last tile done,
//   4 split piece: partial written and counted in, 5 wait for the pair's pieces over,
//   6 share merged, 7 end
// and in slot 8 its piece count (0: no work). Read with ie_prefill_phase_stamps_copy.
#ifdef IE_PREFILL_PHASE_STAMPS
constexpr int PF_STAMP_WGS = 4096;
__device__ unsigned long long pf_phase_stamps[PF_STAMP_WGS * 9];
#define PF_STAMP(i)                                                                            \
    do {                                                                                       \
        if (threadIdx.x == 0 && blockIdx.x < PF_STAMP_WGS)                                     \
            pf_phase_stamps[blockIdx.x * 9 + (i)] = __builtin_amdgcn_s_memrealtime();          \
    } while (0)
#define PF_STAMP_VALUE(i, v)                                                                   \
    do {                                                                                       \
        if (threadIdx.x == 0 && blockIdx.x < PF_STAMP_WGS)                                     \
            pf_phase_stamps[blockIdx.x * 9 + (i)] = (unsigned long long)(v);                   \
    } while (0)
#else
#define PF_STAMP(i) do { } while (0)
#define PF_STAMP_VALUE(i, v) do { } while (0)
#endif

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Workgroup shape: PF_WAVES waves of 32 rows x one query head each, i.e. PF_BM = 16 * PF_WAVES
// packed rows x both query heads of a KV head. 8 waves (one workgroup per CU, 128 rows) halve
// the staging work per MFMA against 4 waves (two workgroups per CU, 64 rows): one staged K/V
// tile serves twice the rows.
#ifndef IE_PREFILL_WAVES
#define IE_PREFILL_WAVES 8
#endif
constexpr int PF_WAVES = IE_PREFILL_WAVES;
static_assert(PF_WAVES == 4 || PF_WAVES == 8, "4 or 8 waves per workgroup");
constexpr int PF_BM = 16 * PF_WAVES;  // packed rows per sub-block
constexpr int PF_BN = 64;             // keys per tile
constexpr int PF_D = 128;
constexpr int PF_THREADS = 64 * PF_WAVES;
constexpr int PF_KP = 512 / PF_THREADS;   // prefix K rows per thread (64 keys x 8 lanes)
constexpr int PF_VK = 1024 / PF_THREADS;  // V keys per thread (64 keys x 16 channel groups)
constexpr int PF_CK = 1024 / PF_THREADS;  // chunk K rows per thread (64 keys x 16 lanes)
constexpr int PF_VG = 64 / PF_VK;         // V key groups (threads per channel group)
#ifndef IE_PREFILL_MAXP
#define IE_PREFILL_MAXP 8
#endif
#ifndef IE_PREFILL_MIN_PIECE_TILES
#define IE_PREFILL_MIN_PIECE_TILES 2
#endif
constexpr int PF_MAXP = IE_PREFILL_MAXP;                        // key pieces per sub-block, at most
constexpr int PF_MIN_PIECE_TILES = IE_PREFILL_MIN_PIECE_TILES;  // tiles per piece, at least
constexpr float RESCALE_SLACK = 8.0f;  // log2 units
#ifndef IE_PREFILL_STRADDLE_MARGIN
#define IE_PREFILL_STRADDLE_MARGIN 2
#endif
constexpr int PF_STRADDLE_MARGIN = IE_PREFILL_STRADDLE_MARGIN;  // tiles

// LDS layouts (bytes), padded so that every fragment address is a per-lane base plus an
// immediate. A fragment read (ds_read_b128, lane (l16, g) at row l16, 16-byte column g) is free of
// bank conflicts on gfx950 when the row stride is 32 mod 64 bytes (measured: strides of 16, 48
// or 0 mod 64 take two passes), hence the 32-byte pads:
//   K tile: row = key, 256 B + 32 B pad; 16-byte unit c (8 channels) at c * 16.
//   V^T tile: row = channel d, 128 B (64 keys) + 32 B pad. Keys are stored in the order the PV
//   MFMA consumes them: within each 32-key half, position 8g + j holds key 4g + j (j < 4) and
//   key 16 + 4g + (j - 4) (j >= 4), so a lane's 8 keys for one 32-key step are one 16-byte read.
constexpr int KS_STRIDE = 288;
constexpr int VT_STRIDE = 160;
constexpr int QS_STRIDE = 288;  // per-wave Q staging rows (see load_q)
__device__ __forceinline__ int ks_off(int key, int c) { return key * KS_STRIDE + (c << 4); }
// byte offset of keys [4kg, 4kg + 4) of channel d
__device__ __forceinline__ int vt_off4(int d, int kg) {
    const int half = kg >> 3, k16 = kg & 7;  // kg: group of 4 keys within the 64-key tile
    const int pos = 32 * half + ((k16 & 3) << 3) + ((k16 >> 2) << 2);
    return d * VT_STRIDE + pos * 2;
}

// Sign-extended byte j of w as float (one v_cvt_f32_i32 with an SDWA byte select).
__device__ __forceinline__ float sbyte(uint32_t w, int j) {
    return (float)((int32_t)(w << (24 - 8 * j)) >> 24);
}
// bf16 pair from two floats whose low 16 bits are zero (exact small integers).
__device__ __forceinline__ uint32_t hi16pair(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// The workgroup's LDS: two K and two V^T tile buffers and three K-scale slots. Before the tile
// loop the second K buffer holds the schedule's entry tables (cu_seqlens, cu_cached and
// slot_ids of up to PF_LDS_ENTRIES entries): no wave writes it before the first barrier of the
// item, which every wave reaches only after its schedule. 79,360 bytes: two workgroups fit a
// CU's 160 KB.
struct PfLds {
    uint8_t k[2][PF_BN * KS_STRIDE];
    uint8_t vt[2][PF_D * VT_STRIDE];
    float ksc[3][PF_BN];
    float kb[3][PF_BN];
#if IE_PREFILL_WAVES == 8
    uint8_t q[PF_WAVES][32 * QS_STRIDE];  // one workgroup per CU: room for separate Q regions
#endif
};

struct PrefillArgs {
    const uint16_t* q;
    int64_t q_st, q_sh;
    const uint16_t* k;
    int64_t k_st, k_sh;
    const uint16_t* v;
    int64_t v_st, v_sh;
    const int32_t* seq_ids;
    const int32_t* cu_seqlens;
    const int32_t* tile_start;
    const int32_t* slot_ids;
    const int32_t* cu_cached;
    ie_kv_cache c;
    uint16_t* out;
    int64_t o_st, o_sh;
    uint16_t* part_o;  // [slot][8 channel blocks][2 heads][PF_BM rows][16] bf16: normalized
                       // partial O of split items, in the accumulators' order (a store of 16
                       // rows x 16 channels is 512 contiguous bytes)
    float* part_ml;    // [slot][2 heads][PF_BM rows][2]: their (m, l)
    const int32_t* plan;  // null, or the launch's work list as ie_prefill_attention_plan writes
                          // it (16 int32 per workgroup): then no workgroup computes it
    uint32_t* arrivals;  // [2][grid]: arrival and finish words of each split (sub-block, kv
                         // head) pair, at the pair's first item; 0 between launches
    uint64_t merge_wait_ticks;   // longest wait of a piece for its pair's others (100 MHz clock)
    uint64_t merge_stall_ticks;  // ... and longest wait with no other piece arriving
    int block_m, sub_per_tile, hq, hkv;
    int ratio;   // query heads per KV head (GQA ratio, 1 ... 16)
    int npairs;  // query-head pairs per KV head, cdiv(ratio, 2)
    int units;   // hkv * npairs: the work items of a (sub-block, piece), one per (KV head, pair)
    int nent;  // entries (length of slot_ids; cu_seqlens and cu_cached hold nent + 1)
    int ntok;  // packed rows (length of seq_ids)
    int nsb;   // sub-blocks: num_tiles * sub_per_tile
    int grid;  // partial slots (resident main-kernel workgroups); split items are numbered below it
    float qk_scale;  // D^-0.5 * log2(e)
};

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Sub-block `sb` (tile sb / sub_per_tile, 64-row slice sb % sub_per_tile) as seen by the calling
// lane: rows [r0, r1) of the entry starting at packed row seq_start, its cache slot and prefix
// length P, and its key tiles: cdiv(P, 64) prefix tiles then cdiv(r1 - seq_start, 64) chunk
// tiles (npt, nct; both 0 when the sub-block has no rows).
struct SbInfo {
    int npt, nct, r0, r1, seq_start, P, slot;
};

constexpr int PF_UNSPLIT = 1 << 28;  // piece size that never splits a pair
constexpr int PF_PLAN_FIELDS = 16;   // int32 per workgroup in an exported work list


// Pieces of a pair with npt prefix and nct chunk tiles at piece size T. A pair of at most T
// tiles is one piece; a longer one is split into prefix pieces and chunk pieces separately (no
// piece mixes the two loops, so none pays two pipeline prologues), evenly within each part, at
// most PF_MAXP pieces in all.
__device__ __forceinline__ int prefix_pieces(int npt, int nct, const Divisor& T) {
    if (npt + nct <= T.d) return 0;
    return npt == 0 ? 0 : min(PF_MAXP - 1, div_ceil(npt, T));
}
__device__ __forceinline__ int piece_count(int npt, int nct, const Divisor& T) {
    if (npt + nct == 0) return 0;
    if (npt + nct <= T.d) return 1;
    const int pp = prefix_pieces(npt, nct, T);
    return pp + min(PF_MAXP - pp, div_ceil(nct, T));
}
// Pieces of a pair in the straddling form: its tiles, prefix then chunk, cut evenly into
// cdiv(n, T) consecutive ranges (at most PF_MAXP); the range that crosses from the prefix into
// the chunk runs both loops.
__device__ __forceinline__ int straddle_count(int ntiles, const Divisor& T) {
    return ntiles == 0 ? 0 : min(PF_MAXP, div_ceil(ntiles, T));
}

// The launch's work list, computed identically by every workgroup from the tile metadata:
//  * piece size T (tiles): a (sub-block, kv head) pair becomes piece_count items. T is the
//    smallest size (at least PF_MIN_PIECE_TILES) whose item count fits the partial slots, so
//    that every split item owns a slot: the search runs from the lower bound
//    cdiv(sum(n) * Hkv, slots) up to the worst-rounding bound, where every part rounds up by a
//    whole piece (sum(n / T) + parts) * Hkv <= slots, which always fits. With more (sub-block
//    part, head) pairs than slots this separate form cannot split. The straddling form
//    (straddle_count) cuts each pair's tiles into even consecutive ranges whatever the parts,
//    so it splits whenever the pairs alone fit the slots: a few sub-blocks over long prefixes
//    (e.g. 16 chunks of 64 tokens each continuing a long context), which the separate form
//    leaves one workgroup per pair on half the CUs. It is used when its pieces are shorter by
//    more than PF_STRADDLE_MARGIN tiles (a piece that crosses into the chunk pays a second
//    loop prologue, about two tiles' time).
//  * items in launch order: sub-blocks from last to first (later sub-blocks of a sequence see
//    more keys), then piece, then kv head.
// schedule(target) finds the sub-block holding item `target`, the offset inside it and the
// number of items before the sub-block. With up to PF_LDS_ENTRIES entries all metadata comes in
// one memory round trip: the tile starts of the wave's sub-blocks (PF_SCHED_CHUNKS * 64 in
// registers, reloaded beyond) and the per-entry tables (cu_seqlens, cu_cached, slot_ids) staged
// in LDS, where each sub-block finds its entry by binary search (an entry owns the rows
// [cu_seqlens[e], cu_seqlens[e + 1]); the largest e with cu_seqlens[e] <= row is that row's
// entry, empty entries included). With more entries (engines with a large max_batch_size) a
// sub-block reads its entry from seq_ids at its tile's first row, as the reference kernel does
// (kernels.py:1029-1033), and that entry's table values from global memory: two more dependent
// round trips, no limit on the entry count.
constexpr int PF_SCHED_CHUNKS = 4;
constexpr int PF_LDS_ENTRIES = 512;

struct SubBlock {
    // npp: prefix pieces, or -1 in the straddling form
    int r0, r1, seq_start, P, slot, npt, nct, ntiles, npieces, npp;
};

__device__ __forceinline__ void fill_sub_block(SubBlock& s, int r0, int r1, int seq_start, int P,
                                               int slot, const Divisor& T, bool straddle) {
    s.r0 = r0;
    s.r1 = r1;
    s.seq_start = seq_start;
    s.P = P;
    s.slot = slot;
    s.npt = cdiv_i(P, PF_BN);
    s.nct = cdiv_i(r1 - seq_start, PF_BN);
    s.ntiles = s.npt + s.nct;
    s.npieces = straddle ? straddle_count(s.ntiles, T) : piece_count(s.npt, s.nct, T);
    s.npp = straddle ? -1 : prefix_pieces(s.npt, s.nct, T);
}

struct Loc {
    int sb, off, item_base, T;
    int found;
    int straddle;
    SubBlock s;       // sub-block sb
};

// One wave's pass over the tile metadata (every lane of the wave returns the same Loc). Every
// wave of the workgroup runs it: each writes the same values into the entry tables in LDS
// (`tables`) before reading them, so no wave waits for another.
__device__ Loc schedule(const PrefillArgs& a, int target, int* tables) {
    static_assert((3 * PF_LDS_ENTRIES + 2) * sizeof(int) <= sizeof(PfLds::k[1]),
                  "entry tables must fit one K buffer");
    int* s_cu = tables;
    int* s_cc = tables + PF_LDS_ENTRIES + 1;
    int* s_sl = tables + 2 * (PF_LDS_ENTRIES + 1);
    const bool in_lds = a.nent <= PF_LDS_ENTRIES;  // uniform
    const int lane = threadIdx.x & 63;
    const int nchunks = cdiv_i(a.nsb, IE_WAVE);
    const Divisor spt = divisor(a.sub_per_tile);
    auto sb_of = [&](int c) { return a.nsb - 1 - (c * IE_WAVE + lane); };
    auto row_start_of = [&](int sb) {
        return sb >= 0 && sb < a.nsb ? a.tile_start[div_floor(sb, spt)] : -1;
    };
    // the round trip: tile starts first, then the entry tables (all independent loads)
    int rs[PF_SCHED_CHUNKS];
#pragma unroll
    for (int c = 0; c < PF_SCHED_CHUNKS; ++c) rs[c] = row_start_of(c < nchunks ? sb_of(c) : -1);
    if (in_lds) {
        for (int e = lane; e <= a.nent; e += IE_WAVE) {
            s_cu[e] = a.cu_seqlens[e];
            s_cc[e] = a.cu_cached[e];
            if (e < a.nent) s_sl[e] = a.slot_ids[e];
        }
    }
    // A workgroup past the slots has no item whenever the slots exceed parts x Hkv (the pairs
    // are then split and every item is numbered below the slots, see below). A sub-block has at
    // most a prefix part and a chunk part, so twice the sub-blocks of tiles with work bound the
    // parts from the tile starts alone: such a workgroup (these start late, once resident ones
    // finish) leaves before the entry lookups.
    if (__builtin_expect(target >= a.grid && nchunks <= PF_SCHED_CHUNKS, 0)) {
        int busy = 0;
#pragma unroll
        for (int c = 0; c < PF_SCHED_CHUNKS; ++c) busy += rs[c] >= 0 ? 1 : 0;
        if (2 * uni(wave_sum_i(busy)) * a.units < a.grid) {
            Loc L;
            L.found = 0;
            L.straddle = 0;
            L.T = 0;
            L.sb = L.off = L.item_base = 0;
            L.s = SubBlock{};
            return L;
        }
    }
    auto info = [&](int sb, int row_start) {
        SbInfo z = {0, 0, 0, 0, 0, 0, 0};
        if (row_start < 0) return z;
        int seq_start, seq_end, P, slot;
        if (in_lds) {
            int lo = 0, hi = a.nent - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_cu[mid] <= row_start) lo = mid;
                else hi = mid - 1;
            }
            seq_start = s_cu[lo];
            seq_end = s_cu[lo + 1];
            P = s_cc[lo + 1] - s_cc[lo];
            slot = s_sl[lo];
        } else {
            // a tile start or entry id out of range reads nothing past the index arrays
            if (row_start >= a.ntok) return z;
            const int e = min(max(a.seq_ids[row_start], 0), a.nent - 1);
            seq_start = a.cu_seqlens[e];
            seq_end = a.cu_seqlens[e + 1];
            P = a.cu_cached[e + 1] - a.cu_cached[e];
            slot = a.slot_ids[e];
        }
        const int sub = sb - div_floor(sb, spt) * a.sub_per_tile;
        const int r0 = row_start + sub * PF_BM;
        const int r1 = min(min(r0 + PF_BM, row_start + a.block_m), seq_end);
        if (r0 >= r1) return z;
        z.P = P;
        z.npt = cdiv_i(z.P, PF_BN);
        z.nct = cdiv_i(r1 - seq_start, PF_BN);
        z.r0 = r0;
        z.r1 = r1;
        z.seq_start = seq_start;
        z.slot = slot;
        return z;
    };
    SbInfo zc[PF_SCHED_CHUNKS];
    int tot = 0, parts = 0;
#pragma unroll
    for (int c = 0; c < PF_SCHED_CHUNKS; ++c) {
        zc[c] = info(c < nchunks ? sb_of(c) : -1, rs[c]);
        tot += zc[c].npt + zc[c].nct;
        parts += (zc[c].npt > 0) + (zc[c].nct > 0);
    }
    for (int c = PF_SCHED_CHUNKS; c < nchunks; ++c) {
        const SbInfo z = info(sb_of(c), row_start_of(sb_of(c)));
        tot += z.npt + z.nct;
        parts += (z.npt > 0) + (z.nct > 0);
    }
    tot = uni(wave_sum_i(tot));
    parts = uni(wave_sum_i(parts));
    // f(z) summed over the launch's sub-blocks (every lane gets the sum)
    auto launch_sum = [&](auto f) {
        int n = 0;
#pragma unroll
        for (int c = 0; c < PF_SCHED_CHUNKS; ++c) n += f(zc[c]);
        for (int c = PF_SCHED_CHUNKS; c < nchunks; ++c) n += f(info(sb_of(c), row_start_of(sb_of(c))));
        return uni(wave_sum_i(n));
    };
    const int spare = a.grid - parts * a.units;
    // the straddling form's lower bound on its piece size; it can only be chosen when its
    // pieces beat the separate form's by PF_STRADDLE_MARGIN tiles and the pairs, one piece
    // each, fit the slots
    int lo = max(PF_MIN_PIECE_TILES, cdiv_i(tot * a.units, a.grid));
    bool straddle_fits = false;
    auto straddle_check = [&]() {
        straddle_fits = launch_sum([](const SbInfo& z) { return z.npt + z.nct > 0 ? 1 : 0; }) *
                            a.units < a.grid;
    };
    if (__builtin_expect(spare <= 0, 0)) straddle_check();
    Loc L;
    L.found = 0;
    L.straddle = 0;
    if ((spare > 0 || straddle_fits) && target >= a.grid) {
        // with spare slots the pairs are split and every item is numbered below a.grid: a
        // workgroup past them has no item (these start late, once resident ones finish, and
        // would otherwise spend the rest of the schedule finding that out)
        L.T = 0;
        L.sb = L.off = L.item_base = 0;
        L.s = SubBlock{};
        return L;
    }
    L.T = PF_UNSPLIT;
    if (spare > 0) {
        L.T = max(PF_MIN_PIECE_TILES, cdiv_i(tot * a.units, spare));
        for (int T = max(PF_MIN_PIECE_TILES, cdiv_i(tot * a.units, a.grid)); T < L.T; ++T) {
            const Divisor D = divisor(T);
            if (launch_sum([&](const SbInfo& z) { return piece_count(z.npt, z.nct, D); }) * a.units <=
                a.grid) {
                L.T = T;
                break;
            }
        }
    }
    // the straddling form's piece size: the smallest T whose pieces fit the slots (binary
    // search: the count falls as T grows, and at the longest pair every pair is one piece,
    // which fits). It replaces the separate form when that is PF_STRADDLE_MARGIN tiles longer
    // (or does not split at all): a crossing piece pays a second loop prologue. Nothing of
    // this runs when even the lower bound cannot win by that margin.
    if (__builtin_expect(spare > 0 && lo + PF_STRADDLE_MARGIN < L.T, 0)) straddle_check();
    if (__builtin_expect(straddle_fits && lo + PF_STRADDLE_MARGIN < L.T, 0)) {
        int hi = lo;
#pragma unroll
        for (int c = 0; c < PF_SCHED_CHUNKS; ++c) hi = max(hi, zc[c].npt + zc[c].nct);
        for (int c = PF_SCHED_CHUNKS; c < nchunks; ++c) {
            const SbInfo z = info(sb_of(c), row_start_of(sb_of(c)));
            hi = max(hi, z.npt + z.nct);
        }
        hi = uni((int)wave_max((float)hi));  // the longest pair (< 2^24 tiles: exact)
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            const Divisor D = divisor(mid);
            if (launch_sum([&](const SbInfo& z) { return straddle_count(z.npt + z.nct, D); }) *
                    a.units <= a.grid)
                hi = mid;
            else
                lo = mid + 1;
        }
        if (lo + PF_STRADDLE_MARGIN < L.T) {
            L.T = lo;
            L.straddle = 1;
        }
    }
    const Divisor DT = divisor(L.T);
    const bool straddle = L.straddle != 0;
    int np[PF_SCHED_CHUNKS];  // pieces of the lane's sub-blocks
#pragma unroll
    for (int c = 0; c < PF_SCHED_CHUNKS; ++c)
        np[c] = straddle ? straddle_count(zc[c].npt + zc[c].nct, DT)
                         : piece_count(zc[c].npt, zc[c].nct, DT);
    L.found = 0;
    L.sb = L.off = L.item_base = 0;
    int items_before = 0;
    auto visit = [&](int c, const SbInfo& z, int np) {
        const int items = np * a.units;
        const int incl = wave_incl_scan_i(items) + items_before;
        const unsigned long long hit = __ballot(target < incl && target >= incl - items);
        if (hit) {
            const int src = __builtin_ctzll(hit);  // the same lane in every wave: uniform
            auto from = [&](int x) { return __builtin_amdgcn_readlane(x, src); };
            L.sb = from(sb_of(c));
            L.item_base = from(incl - items);
            L.off = target - L.item_base;
            fill_sub_block(L.s, from(z.r0), from(z.r1), from(z.seq_start), from(z.P),
                           from(z.slot), DT, straddle);
            L.found = 1;
        }
        items_before = __builtin_amdgcn_readlane(incl, 63);
        return L.found != 0;
    };
#pragma unroll
    for (int c = 0; c < PF_SCHED_CHUNKS; ++c)
        if (c < nchunks && visit(c, zc[c], np[c])) return L;
    for (int c = PF_SCHED_CHUNKS; c < nchunks; ++c) {
        const SbInfo z = info(sb_of(c), row_start_of(sb_of(c)));
        if (visit(c, z, straddle ? straddle_count(z.npt + z.nct, DT)
                                 : piece_count(z.npt, z.nct, DT)))
            return L;
    }
    return L;
}

// Global data of one tile, held in registers between its load and its LDS staging.
// Buffer descriptors of one (sub-block, kv head): prefix K/V rows (128 B each, P rows) and scales
// of the cache, and the chunk's bf16 K/V rows [seq_start, r1). Reads past those ranges return 0.
struct TileSrc {
    rsrc_t pk, pv, pks, pvs, ck, cv;
    int ck_stride, cv_stride;  // bytes between chunk rows
};

__device__ __forceinline__ u32x4 ld128(rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ u32x2 ld64(rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ float ldf(rsrc_t r, int off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Prefix tiles, K and V handled separately (the prefix loop stages K two tiles and V one tile
// ahead of the MFMAs): the int8 rows and per-key scales of one tile, in registers between load
// and staging. K is staged as exact bf16 integers (its scale multiplies the scores); V is staged
// dequantized, bf16(v * v_scale), the rounding the reference's dequantization applies, so P
// needs no per-key factor.
// K rows are loaded 8 lanes per 128-byte row (thread: keys (tid >> 3) + i * PF_THREADS / 8,
// channels [16 (tid & 7), +16)): wave loads that cover few lanes per row moved a third of the
// bytes per clock on this part. V: thread (key group kg = tid % PF_VG, channel group
// dg = tid / PF_VG) holds channels [8 dg, +8) of keys PF_VK kg + u.
struct PfxK {
    u32x4 kw[PF_KP];
    float kscale, kbias;
};
struct PfxV {
    u32x2 vw[PF_VK];
    float vs[PF_VK];  // v_scale of the thread's keys (0 past P: out of the buffer range)
};
__device__ __forceinline__ void load_pk(PfxK& r, const TileSrc& src, int kbase, int P) {
    const int tid = threadIdx.x;
    const int off = (kbase + (tid >> 3)) * PF_D + 16 * (tid & 7);
#pragma unroll
    for (int i = 0; i < PF_KP; ++i) r.kw[i] = ld128(src.pk, off + i * (PF_THREADS / 8) * PF_D);
    const int kk = kbase + (tid & (PF_BN - 1));
    r.kscale = ldf(src.pks, 4 * kk);
    r.kbias = kk < P ? 0.f : -INFINITY;
}
__device__ __forceinline__ void load_pv(PfxV& r, const TileSrc& src, int kbase) {
    const int tid = threadIdx.x;
    const int kg = tid % PF_VG, dg = tid / PF_VG;
#pragma unroll
    for (int u = 0; u < PF_VK; ++u)
        r.vw[u] = ld64(src.pv, (kbase + PF_VK * kg + u) * PF_D + 8 * dg);
    if constexpr (PF_VK == 4) {
        const f32x4 v = __builtin_bit_cast(f32x4, ld128(src.pvs, 4 * (kbase + 4 * kg)));
#pragma unroll
        for (int u = 0; u < 4; ++u) r.vs[u] = v[u];
    } else {
        const u32x2 v = ld64(src.pvs, 4 * (kbase + PF_VK * kg));
        r.vs[0] = __uint_as_float(v[0]);
        r.vs[1] = __uint_as_float(v[1]);
    }
}
// byte offset in a V^T tile of the PF_VK keys [PF_VK kg, +PF_VK) of channel d (consecutive
// positions of the MFMA key order)
__device__ __forceinline__ int vt_off_keys(int d, int kg) {
    return vt_off4(d, (PF_VK * kg) >> 2) + 2 * ((PF_VK * kg) & 3);
}
// 16 int8 channels -> two 16-byte bf16 units 2c and 2c + 1 of the key's row, the one written
// first alternating with c / 4 so that each 8-lane store group covers distinct banks.
__device__ __forceinline__ void stage_pk(const PfxK& r, uint8_t* s_k) {
    const int tid = threadIdx.x, c = tid & 7, sw = (c >> 2) & 1;
#pragma unroll
    for (int i = 0; i < PF_KP; ++i) {
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            w[2 * j] = hi16pair(sbyte(r.kw[i][j], 0), sbyte(r.kw[i][j], 1));
            w[2 * j + 1] = hi16pair(sbyte(r.kw[i][j], 2), sbyte(r.kw[i][j], 3));
        }
        uint8_t* row = s_k + ks_off((tid >> 3) + i * (PF_THREADS / 8), 2 * c);
        const u32x4 lo = {w[0], w[1], w[2], w[3]}, hi = {w[4], w[5], w[6], w[7]};
        *reinterpret_cast<u32x4*>(row + 16 * sw) = sw ? hi : lo;
        *reinterpret_cast<u32x4*>(row + 16 * (1 - sw)) = sw ? lo : hi;
    }
}
__device__ __forceinline__ void stage_pk_scales(const PfxK& r, float* s_ksc, float* s_kb,
                                                float qk_scale) {
    const int tid = threadIdx.x;
    if (tid < PF_BN) {
        s_ksc[tid] = r.kscale * qk_scale;
        s_kb[tid] = r.kbias;
    }
}
__device__ __forceinline__ void stage_pv(const PfxV& r, uint8_t* s_vt) {
    const int tid = threadIdx.x;
    const int kg = tid % PF_VG, dg = tid / PF_VG;
    uint8_t* dst = s_vt + vt_off_keys(8 * dg, kg);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int wj = j >> 2, bj = j & 3;
        const uint32_t p01 = pack_bf16x2(sbyte(r.vw[0][wj], bj) * r.vs[0], sbyte(r.vw[1][wj], bj) * r.vs[1]);
        if constexpr (PF_VK == 4) {
            const uint32_t p23 = pack_bf16x2(sbyte(r.vw[2][wj], bj) * r.vs[2], sbyte(r.vw[3][wj], bj) * r.vs[3]);
            *reinterpret_cast<u32x2*>(dst + j * VT_STRIDE) = u32x2{p01, p23};
        } else {
            *reinterpret_cast<uint32_t*>(dst + j * VT_STRIDE) = p01;
        }
    }
}

// Chunk tiles: bf16 rows seq_start + [kbase, kbase + 64) of the packed chunk (zeros at or past
// the sub-block's last row: the buffer range does the masking), K and V in registers between
// load and staging. V has the prefix tiles' lane mapping.
struct ChkK {
    u32x4 w[PF_CK];  // keys (tid >> 4) + i PF_THREADS / 16, channels [8 (tid & 15), +8): 16 lanes
                     // per 256-byte row
};
struct ChkV {
    u32x4 w[PF_VK];  // keys PF_VK (tid % PF_VG) + u, channels [8 (tid / PF_VG), +8)
};
__device__ __forceinline__ void load_ck(ChkK& r, const TileSrc& src, int kbase) {
    const int tid = threadIdx.x;
    const int off = (kbase + (tid >> 4)) * src.ck_stride + 16 * (tid & 15);
#pragma unroll
    for (int i = 0; i < PF_CK; ++i)
        r.w[i] = ld128(src.ck, off + i * (PF_THREADS / 16) * src.ck_stride);
}
__device__ __forceinline__ void load_cv(ChkV& r, const TileSrc& src, int kbase) {
    const int tid = threadIdx.x;
    const int kg = tid % PF_VG, dg = tid / PF_VG;
#pragma unroll
    for (int u = 0; u < PF_VK; ++u)
        r.w[u] = ld128(src.cv, (kbase + PF_VK * kg + u) * src.cv_stride + 16 * dg);
}
__device__ __forceinline__ void stage_ck(const ChkK& r, uint8_t* s_k) {
    const int tid = threadIdx.x;
    uint8_t* dst = s_k + ks_off(tid >> 4, tid & 15);
#pragma unroll
    for (int i = 0; i < PF_CK; ++i)
        *reinterpret_cast<u32x4*>(dst + i * (PF_THREADS / 16) * KS_STRIDE) = r.w[i];
}
__device__ __forceinline__ void stage_cv(const ChkV& r, uint8_t* s_vt) {
    const int tid = threadIdx.x;
    uint8_t* dst = s_vt + vt_off_keys(8 * (tid / PF_VG), tid % PF_VG);
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // channel j of key u: bf16 half (j & 1) of word j >> 1
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t p01 = __builtin_amdgcn_perm(r.w[1][j >> 1], r.w[0][j >> 1], sel);
        if constexpr (PF_VK == 4) {
            const uint32_t p23 = __builtin_amdgcn_perm(r.w[3][j >> 1], r.w[2][j >> 1], sel);
            *reinterpret_cast<u32x2*>(dst + j * VT_STRIDE) = u32x2{p01, p23};
        } else {
            *reinterpret_cast<uint32_t*>(dst + j * VT_STRIDE) = p01;
        }
    }
}

// Per-wave running state: O^T accumulators (lane: d = 16mt + 4g + i, row = 16nt + l16) and the
// base-2 running max / sum of the lane's two rows.
// Per row tile nt (the lane's row l16 of it): the running max m, kept as nmb = -m (0 while the
// row has seen no key), and the running sum l of the bf16 probabilities, accumulated by an MFMA
// of a ones matrix with P^T (every element of lsum[nt] holds the lane's row sum).
struct WaveState {
    f32x4 acc[8][2];
    f32x4 lsum[2];
    float nmb[2];
};

// Tile kinds for the score scaling: prefix tiles (scores scaled per key) that are full or hold
// keys past P (masked through the staged -inf bias); chunk tiles (one scale; the causal mask is
// applied in softmax_rescale).
enum : int { TILE_PREFIX = 0, TILE_PREFIX_PARTIAL = 1, TILE_CHUNK = 2 };

// The three parts of one wave's work on a staged 64-key tile (the sum is tile_compute):
//   tile_scores   S^T = K . Q^T, 64 keys x 32 rows, 32 MFMAs (4 steps of 16 keys)
//   softmax       scale, mask, online softmax (base 2) -> P^T as bf16 MFMA B fragments
//   tile_pv       O^T += V^T . P^T, 32 MFMAs
// Chunk key c is visible to row m iff seq_start + c <= m and c < r1 - seq_start (lim0 / lim1:
// last visible key of the lane's two rows).

// One 16-key step of S^T: reads the step's K fragments and runs the two 4-MFMA chains.
__device__ __forceinline__ void score_step(f32x4 (&st)[4][2], const bf16x8 (&qf)[2][4],
                                           const uint8_t* kfrag, int mt) {
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    bf16x8 kf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        kf[ks] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u32x4*>(kfrag + 16 * mt * KS_STRIDE + 64 * ks));
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[0], qf[nt][0], zero4, 0, 0, 0);
#pragma unroll
        for (int ks = 1; ks < 4; ++ks)
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[nt][ks], c, 0, 0, 0);
        st[mt][nt] = c;
    }
}

__device__ __forceinline__ void tile_scores(f32x4 (&st)[4][2], const bf16x8 (&qf)[2][4],
                                            const uint8_t* s_k, int l16, int g) {
    // fragment reads run one 16-key step ahead of the MFMAs that consume them
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const uint8_t* kfrag = s_k + ks_off(l16, g);
    auto read_k = [&](bf16x8 (&kf)[4], int mt) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            kf[ks] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(kfrag + 16 * mt * KS_STRIDE + 64 * ks));
    };
    bf16x8 kf[2][4];
    read_k(kf[0], 0);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        __builtin_amdgcn_sched_barrier(0);
        if (mt < 3) read_k(kf[(mt + 1) & 1], mt + 1);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[mt & 1][0], qf[nt][0], zero4, 0, 0, 0);
#pragma unroll
            for (int ks = 1; ks < 4; ++ks)
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[mt & 1][ks], qf[nt][ks], c, 0, 0, 0);
            st[mt][nt] = c;
        }
    }
}

// Softmax part 1 for row tile nt: scale (relative to the running max), the prefix-partial mask,
// and the max over the lane's own 16 keys of the tile (the row's max needs the other three lanes
// of the row only when the running max moves). Branch-free.
template <int KIND>
__device__ __forceinline__ float softmax_scale(f32x4 (&st)[4][2], int nt, float nmb,
                                               const float* s_ksc, const float* s_kb,
                                               float qk_scale, int g) {
    constexpr bool PREFIX = KIND == TILE_PREFIX || KIND == TILE_PREFIX_PARTIAL;
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        f32x4 ksv = {qk_scale, qk_scale, qk_scale, qk_scale};
        if (PREFIX) ksv = *reinterpret_cast<const f32x4*>(s_ksc + 16 * mt + 4 * g);
        f32x4 kbv = {0.f, 0.f, 0.f, 0.f};
        if (KIND == TILE_PREFIX_PARTIAL) kbv = *reinterpret_cast<const f32x4*>(s_kb + 16 * mt + 4 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float x = __builtin_fmaf(st[mt][nt][i], ksv[i], nmb);
            if (KIND == TILE_PREFIX_PARTIAL) x += kbv[i];  // -inf past P
            st[mt][nt][i] = x;
            mx = fmaxf(mx, x);
        }
    }
    return mx;
}

// Softmax part 2 for row tile nt: the lazy running max. It moves only when the row's tile max
// exceeds it by more than RESCALE_SLACK, so probabilities stay <= 2^RESCALE_SLACK, and it is set
// on the first tile of a work item. A row that sees no key of an item's first tile sees none of
// its later tiles either (prefix tiles are visible to every row and chunk tiles come in causal
// order), so that first tile (`first`, wave-uniform) is the only place where a row's first key
// can appear. The common path is one compare of the lane's own max; in the rare, wave-uniform
// branch the row's max is reduced over its four lanes (every lane of a row takes the same
// decision), the wave shifts its scores once more and rescales the accumulators.
// Chunk tiles on the causal diagonal or past the sub-block's last row (`diag`, wave-uniform: at
// most two per wave and item) take the rare branch too, which masks them first (chunk key
// kbase + 16mt + 4g + i is visible to the lane's row iff it is <= lim).
__device__ __forceinline__ void softmax_rescale(WaveState& w, f32x4 (&st)[4][2], int nt,
                                                float mx, bool first, bool diag = false,
                                                int kbase = 0, int lim = 0, int g = 0) {
    if (first || diag || __ballot(mx > RESCALE_SLACK)) {
        if (diag) {
            mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x = kbase + 16 * mt + 4 * g + i <= lim ? st[mt][nt][i] : -INFINITY;
                    st[mt][nt][i] = x;
                    mx = fmaxf(mx, x);
                }
        }
        const float rmx = max_xor32(max_xor16(mx));
        const bool move = first ? rmx != -INFINITY : rmx > RESCALE_SLACK;
        const float shift = move ? rmx : 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) st[mt][nt] -= shift;
        w.nmb[nt] -= shift;
        if (!first) {  // before the first tile, l and the accumulators are 0
            const float alpha = __builtin_amdgcn_exp2f(-shift);  // 1 unless moved
            w.lsum[nt] *= alpha;
            if (__ballot(move)) {
#pragma unroll
                for (int mt = 0; mt < 8; ++mt) w.acc[mt][nt] *= alpha;
            }
        }
    }
}

// Softmax part 3 for row tile nt: probabilities as bf16 P^T fragments. Branch-free.
__device__ __forceinline__ void softmax_p(const f32x4 (&st)[4][2], int nt,
                                          uint32_t (&pfrag)[2][2][4]) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; i += 2)
            pfrag[mt >> 1][nt][(mt & 1) * 2 + i / 2] =
                pack_bf16x2(__builtin_amdgcn_exp2f(st[mt][nt][i]),
                            __builtin_amdgcn_exp2f(st[mt][nt][i + 1]));
}

// O^T += V^T . P^T (32 MFMAs) and the row sums l += ones . P^T (4 MFMAs: the row sum lands in
// all four elements of lsum[nt], and it is the sum of the bf16 probabilities the PV product
// weights, so O / l stays a weighted mean of V rows).
template <bool FENCE = true>
__device__ __forceinline__ void tile_pv(WaveState& w, const uint32_t (&pfrag)[2][2][4],
                                        const uint8_t* s_vt, int l16, int g) {
    const uint8_t* vfrag = s_vt + l16 * VT_STRIDE + 16 * g;
    auto read_v = [&](bf16x8 (&vf)[2], int mt) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
            vf[s2] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(vfrag + 16 * mt * VT_STRIDE + 64 * s2));
    };
    auto pfv = [&](int s2, int nt) {
        return __builtin_bit_cast(bf16x8, u32x4{pfrag[s2][nt][0], pfrag[s2][nt][1],
                                                pfrag[s2][nt][2], pfrag[s2][nt][3]});
    };
    const bf16x8 ones = __builtin_bit_cast(
        bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
    bf16x8 vf[2][2];
    read_v(vf[0], 0);
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
        if (FENCE) __builtin_amdgcn_sched_barrier(0);
        if (mt < 7) read_v(vf[(mt + 1) & 1], mt + 1);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                w.acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[mt & 1][s2], pfv(s2, nt),
                                                                       w.acc[mt][nt], 0, 0, 0);
        if (mt == 0) {
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    w.lsum[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pfv(s2, nt),
                                                                        w.lsum[nt], 0, 0, 0);
        }
    }
}

// Q^T fragments of this wave: lane holds q[row = wr0 + 16nt + l16][d = 32ks + 8g .. +7], as
// bf16(q * cal) for prefix tiles or bf16 q for chunk tiles; zero rows past the sub-block.
// The 32 rows x 256 bytes are loaded 16 lanes per row (loads in the fragment layout, 16 rows x
// 64 bytes per wave instruction, moved a third of the bytes per clock) into the wave's own LDS
// region `qreg` (rows of QS_STRIDE bytes, 32 mod 64: conflict-free fragment reads) and read back
// in the fragment layout (q_frags). With 8-wave workgroups the region is the wave's own and
// keeps the raw rows; with 4-wave ones it lies in the V^T buffers: the caller keeps them
// unstaged until every wave has passed a barrier after this call.
static_assert(PF_WAVES == 8 || PF_WAVES * 32 * QS_STRIDE <= 2 * PF_D * VT_STRIDE,
              "Q regions must fit the V^T buffers");
template <bool PREFIX>
__device__ __forceinline__ void q_frags(bf16x8 (&qf)[2][4], const float* cal, int l16, int g,
                                        const uint8_t* qreg) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4 w = *reinterpret_cast<const u32x4*>(qreg + (16 * nt + l16) * QS_STRIDE +
                                                      16 * (4 * ks + g));
            if (PREFIX) {
                const f32x4 c0 = *reinterpret_cast<const f32x4*>(cal + 32 * ks + 8 * g);
                const f32x4 c1 = *reinterpret_cast<const f32x4*>(cal + 32 * ks + 8 * g + 4);
                w = u32x4{pack_bf16x2(bf16lo(w.x) * c0[0], bf16hi(w.x) * c0[1]),
                          pack_bf16x2(bf16lo(w.y) * c0[2], bf16hi(w.y) * c0[3]),
                          pack_bf16x2(bf16lo(w.z) * c1[0], bf16hi(w.z) * c1[1]),
                          pack_bf16x2(bf16lo(w.w) * c1[2], bf16hi(w.w) * c1[3])};
            }
            qf[nt][ks] = __builtin_bit_cast(bf16x8, w);
        }
    }
}
template <bool PREFIX>
__device__ __forceinline__ void load_q(bf16x8 (&qf)[2][4], const PrefillArgs& a, int wr0, int r1,
                                       int h, const float* cal, int l16, int g, uint8_t* qreg) {
    const int lane = threadIdx.x & 63, qr = lane >> 4, qc = lane & 15;
#pragma unroll
    for (int half = 0; half < 2; ++half) {  // 16 rows at a time: fewer registers in flight
        u32x4 raw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = wr0 + 16 * half + 4 * j + qr;
            raw[j] = u32x4{0u, 0u, 0u, 0u};
            if (row < r1)
                raw[j] = *reinterpret_cast<const u32x4*>(a.q + row * a.q_st + h * a.q_sh + 8 * qc);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<u32x4*>(qreg + (16 * half + 4 * j + qr) * QS_STRIDE + 16 * qc) = raw[j];
    }
    q_frags<PREFIX>(qf, cal, l16, g, qreg);
}

#ifndef IE_PREFILL_WG_PER_CU
#define IE_PREFILL_WG_PER_CU (8 / IE_PREFILL_WAVES)
#endif

__device__ __forceinline__ void merge_pieces(const PrefillArgs& a, const SubBlock& s, int unit,
                                             int item_base);

// The (KV head, query-head pair) of work-item unit `unit`: KV head hk, query heads qh0 and
// qh0 + 1, the second present unless it is an odd ratio's last pair (has2 false: that wave
// computes a copy of the first head and stores nothing).
struct PfUnit {
    int hk, qh0;
    bool has2;
};
__device__ __forceinline__ PfUnit pf_unit(const PrefillArgs& a, int unit) {
    if (a.npairs == 1) return PfUnit{unit, unit * a.ratio, a.ratio == 2};
    const int hk = uni(unit / a.npairs), pair = unit - hk * a.npairs;
    return PfUnit{hk, uni(a.ratio * hk + 2 * pair), 2 * pair + 1 < a.ratio};
}

// Tiles [kt_begin, kt_end) of piece `piece` of sub-block s (tile kt < npt: prefix tile kt,
// else chunk tile kt - npt): the whole pair, a prefix piece, a chunk piece, or in the
// straddling form an even share of all the pair's tiles.
__device__ __forceinline__ void piece_tiles(const SubBlock& s, int piece, int& kt_begin,
                                            int& kt_end) {
    kt_begin = 0;
    kt_end = s.ntiles;
    if (s.npieces > 1 && s.npp < 0) {
        kt_begin = piece * s.ntiles / s.npieces;
        kt_end = (piece + 1) * s.ntiles / s.npieces;
    } else if (s.npieces > 1) {
        const int q = piece - s.npp, nc = s.npieces - s.npp;
        kt_begin = q < 0 ? piece * s.npt / s.npp : s.npt + q * s.nct / nc;
        kt_end = q < 0 ? (piece + 1) * s.npt / s.npp : s.npt + (q + 1) * s.nct / nc;
    }
}

// One work item: tiles [kt_begin, kt_end) of sub-block s (one of its pieces) for unit `unit`.
__device__ __forceinline__ void prefill_item(const PrefillArgs& a, const SubBlock& s, int unit,
                                             int kt_begin, int kt_end, int item, int item_base,
                                             PfLds& lds) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const PfUnit U = pf_unit(a, unit);
    const int hk = U.hk;
    const bool stores = U.has2 || (wave & 1) == 0;  // this wave's head exists
    const int h = U.has2 ? U.qh0 + (wave & 1) : U.qh0;
    const int wr0 = s.r0 + 32 * (wave >> 1);  // first row of this wave

    // two tile buffers: tile i is staged into buffer i & 1 while the other one is computed on;
    // 3 K-scale slots: the prefix loop rotates them
    auto& s_k = lds.k;
    auto& s_vt = lds.vt;
#if IE_PREFILL_WAVES == 8
    uint8_t* qreg = lds.q[wave];  // this wave's Q staging region
#else
    uint8_t* qreg = &lds.vt[0][0] + wave * 32 * QS_STRIDE;  // this wave's Q staging region
#endif
    auto& s_ksc = lds.ksc;
    auto& s_kb = lds.kb;

    const float* cal = a.c.k_calibration + s.slot * a.c.cal_stride_slot + hk * a.c.cal_stride_head;
    TileSrc src;
    {
        const int64_t crow = s.slot * a.c.stride_slot + hk * a.c.stride_head;
        const int64_t srow = s.slot * a.c.scale_stride_slot + hk * a.c.scale_stride_head;
        src.pk = make_rsrc(a.c.k + crow, (uint32_t)s.P * PF_D);
        src.pv = make_rsrc(a.c.v + crow, (uint32_t)s.P * PF_D);
        src.pks = make_rsrc(a.c.k_scale + srow, (uint32_t)s.P * 4);
        src.pvs = make_rsrc(a.c.v_scale + srow, (uint32_t)s.P * 4);
        const int nrows = s.r1 - s.seq_start;  // chunk rows visible to this sub-block
        src.ck_stride = (int)a.k_st * 2;
        src.cv_stride = (int)a.v_st * 2;
        src.ck = make_rsrc(a.k + s.seq_start * a.k_st + hk * a.k_sh, (uint32_t)(nrows * src.ck_stride));
        src.cv = make_rsrc(a.v + s.seq_start * a.v_st + hk * a.v_sh, (uint32_t)(nrows * src.cv_stride));
    }

    // chunk tiles: last visible chunk key of each of this lane's two rows
    const int rowA = wr0 + l16, rowB = wr0 + 16 + l16;
    const int clim = s.r1 - s.seq_start - 1;
    const int lim0 = min(rowA - s.seq_start, clim), lim1 = min(rowB - s.seq_start, clim);

    // tile kt of the item: prefix tile kt (keys [64kt, ..)) if kt < npt, else chunk tile kt - npt
    WaveState ws;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) ws.acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    ws.lsum[0] = ws.lsum[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    ws.nmb[0] = ws.nmb[1] = 0.f;

    bf16x8 qf[2][4];
    int kt = kt_begin;
    const int prefix_end = min(kt_end, s.npt);
    if (kt < prefix_end) {
        // Prefix tiles, software-pipelined per wave: in step j the MFMAs of S_{j+1} run beside
        // the softmax of tile j, and the PV MFMAs of tile j beside the staging of K_{j+2} and
        // V_{j+1}, whose loads were issued one step earlier. K data buffers alternate (K_j is
        // last read by S_j one step earlier), V buffers alternate, the K scales rotate over
        // three slots (tile j's are read by its softmax while K_{j+2}'s are written).
        const int n = prefix_end - kt, kb0 = kt * PF_BN;
        PfxK pk;
        PfxV pv;
        {
            PfxK pk1;
            load_pk(pk, src, kb0, s.P);
            load_pv(pv, src, kb0);
            if (n > 1) load_pk(pk1, src, kb0 + PF_BN, s.P);
            load_q<true>(qf, a, wr0, s.r1, h, cal, l16, g, qreg);
            stage_pk(pk, s_k[0]);
            stage_pk_scales(pk, s_ksc[0], s_kb[0], a.qk_scale);
            __syncthreads();  // every wave has read its Q region (in the V^T buffers)
            stage_pv(pv, s_vt[0]);
            if (n > 1) {
                stage_pk(pk1, s_k[1]);
                stage_pk_scales(pk1, s_ksc[1], s_kb[1], a.qk_scale);
            }
        }
        if (n > 2) load_pk(pk, src, kb0 + 2 * PF_BN, s.P);
        if (n > 1) load_pv(pv, src, kb0 + PF_BN);
        __syncthreads();
        f32x4 sc[4][2];
        tile_scores(sc, qf, s_k[0], l16, g);
        __syncthreads();  // every wave has read K_0 before step 0 stages K_2 over it
        PF_STAMP(2);
        uint32_t pfrag[2][2][4];
        int slot = 0;  // K-scale slot of tile j
        for (int j = 0; j < n - 1; ++j) {
            const int nslot = slot == 2 ? 0 : slot + 1, fslot = nslot == 2 ? 0 : nslot + 1;
            const uint8_t* kfrag = s_k[(j + 1) & 1] + ks_off(l16, g);
            f32x4 sn[4][2];
            score_step(sn, qf, kfrag, 0);
            score_step(sn, qf, kfrag, 1);
            const float mx0 =
                softmax_scale<TILE_PREFIX>(sc, 0, ws.nmb[0], s_ksc[slot], s_kb[slot], a.qk_scale, g);
            const float mx1 =
                softmax_scale<TILE_PREFIX>(sc, 1, ws.nmb[1], s_ksc[slot], s_kb[slot], a.qk_scale, g);
            softmax_rescale(ws, sc, 0, mx0, j == 0);
            softmax_rescale(ws, sc, 1, mx1, j == 0);
            score_step(sn, qf, kfrag, 2);
            score_step(sn, qf, kfrag, 3);
            softmax_p(sc, 0, pfrag);
            softmax_p(sc, 1, pfrag);
            // PV and the staging of the next tiles in one scheduling region (no fences, no
            // branches), so the conversions fill the MFMA issue gaps
            tile_pv<false>(ws, pfrag, s_vt[j & 1], l16, g);
            stage_pk(pk, s_k[j & 1]);  // K_{j+2}; a harmless copy of stale data if j + 2 == n
            stage_pv(pv, s_vt[(j + 1) & 1]);
            if (j + 2 < n) stage_pk_scales(pk, s_ksc[fslot], s_kb[fslot], a.qk_scale);
            if (j + 3 < n) load_pk(pk, src, kb0 + (j + 3) * PF_BN, s.P);
            if (j + 2 < n) load_pv(pv, src, kb0 + (j + 2) * PF_BN);
            __syncthreads();
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                sc[mt][0] = sn[mt][0];
                sc[mt][1] = sn[mt][1];
            }
            slot = nslot;
        }
        // the last prefix tile of the piece (the only one that can hold keys past P)
        const int j = n - 1;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const float mx = softmax_scale<TILE_PREFIX_PARTIAL>(sc, nt, ws.nmb[nt], s_ksc[slot],
                                                                s_kb[slot], a.qk_scale, g);
            softmax_rescale(ws, sc, nt, mx, n == 1);
            softmax_p(sc, nt, pfrag);
        }
        tile_pv(ws, pfrag, s_vt[j & 1], l16, g);
        __syncthreads();  // the chunk tiles reuse the buffers
        kt = prefix_end;
    }
    if (kt < kt_end) {
        // Chunk tiles, pipelined like the prefix tiles (K_{j+2} and V_{j+1} staged in step j).
        // Tiles that every row of the wave sees whole take the common softmax path; the wave's
        // diagonal tiles (and a last tile past the sub-block's rows) are masked in the rare one.
        const int n = kt_end - kt, kb0 = (kt - s.npt) * PF_BN;
        const int wlim = min(wr0 - s.seq_start, clim);  // keys <= wlim: visible to all rows
        const bool item_start = kt == kt_begin;
        ChkK ck;
        ChkV cv;
        {
            ChkK ck1;
            load_ck(ck, src, kb0);
            load_cv(cv, src, kb0);
            if (n > 1) load_ck(ck1, src, kb0 + PF_BN);
#if IE_PREFILL_WAVES == 8
            // a piece that ran the prefix loop: the raw Q rows are still in this wave's own LDS
            // region, so the chunk loop's fragments need no second global load
            if (kt > kt_begin)
                q_frags<false>(qf, cal, l16, g, qreg);
            else
#endif
                load_q<false>(qf, a, wr0, s.r1, h, cal, l16, g, qreg);
            stage_ck(ck, s_k[0]);
            __syncthreads();  // every wave has read its Q region (in the V^T buffers)
            stage_cv(cv, s_vt[0]);
            if (n > 1) stage_ck(ck1, s_k[1]);
        }
        if (n > 2) load_ck(ck, src, kb0 + 2 * PF_BN);
        if (n > 1) load_cv(cv, src, kb0 + PF_BN);
        __syncthreads();
        f32x4 sc[4][2];
        tile_scores(sc, qf, s_k[0], l16, g);
        __syncthreads();  // every wave has read K_0 before step 0 stages K_2 over it
        if (item_start) PF_STAMP(2);
        uint32_t pfrag[2][2][4];
        for (int j = 0; j < n - 1; ++j) {
            const int kc = kb0 + j * PF_BN;
            const bool diag = kc + PF_BN - 1 > wlim, first = item_start && j == 0;
            const uint8_t* kfrag = s_k[(j + 1) & 1] + ks_off(l16, g);
            f32x4 sn[4][2];
            score_step(sn, qf, kfrag, 0);
            score_step(sn, qf, kfrag, 1);
            const float mx0 = softmax_scale<TILE_CHUNK>(sc, 0, ws.nmb[0], nullptr, nullptr,
                                                        a.qk_scale, g);
            const float mx1 = softmax_scale<TILE_CHUNK>(sc, 1, ws.nmb[1], nullptr, nullptr,
                                                        a.qk_scale, g);
            softmax_rescale(ws, sc, 0, mx0, first, diag, kc, lim0, g);
            softmax_rescale(ws, sc, 1, mx1, first, diag, kc, lim1, g);
            score_step(sn, qf, kfrag, 2);
            score_step(sn, qf, kfrag, 3);
            softmax_p(sc, 0, pfrag);
            softmax_p(sc, 1, pfrag);
            tile_pv<false>(ws, pfrag, s_vt[j & 1], l16, g);
            stage_ck(ck, s_k[j & 1]);  // K_{j+2}; a harmless copy of stale data if j + 2 == n
            stage_cv(cv, s_vt[(j + 1) & 1]);
            if (j + 3 < n) load_ck(ck, src, kb0 + (j + 3) * PF_BN);
            if (j + 2 < n) load_cv(cv, src, kb0 + (j + 2) * PF_BN);
            __syncthreads();
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                sc[mt][0] = sn[mt][0];
                sc[mt][1] = sn[mt][1];
            }
        }
        const int kc = kb0 + (n - 1) * PF_BN;
        const bool diag = kc + PF_BN - 1 > wlim, first = item_start && n == 1;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const float mx = softmax_scale<TILE_CHUNK>(sc, nt, ws.nmb[nt], nullptr, nullptr,
                                                       a.qk_scale, g);
            softmax_rescale(ws, sc, nt, mx, first, diag, kc, nt ? lim1 : lim0, g);
            softmax_p(sc, nt, pfrag);
        }
        tile_pv(ws, pfrag, s_vt[(n - 1) & 1], l16, g);
    }
    PF_STAMP(3);
    // ---- results: lane holds row = wr0 + 16nt + l16, channels d = 16mt + 4g + i ----
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float l = ws.lsum[nt][0];
        const int row = wr0 + 16 * nt + l16;
        if (row >= s.r1 || !stores) continue;
        const float rl = l != 0.f ? 1.f / l : 0.f;
        if (s.npieces == 1) {
            uint16_t* o = a.out + row * a.o_st + h * a.o_sh;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) {
                const f32x4 x = ws.acc[mt][nt];
                *reinterpret_cast<u32x2*>(o + 16 * mt + 4 * g) =
                    u32x2{pack_bf16x2(x[0] * rl, x[1] * rl), pack_bf16x2(x[2] * rl, x[3] * rl)};
            }
        } else {  // normalized partial O in bf16 (a weighted mean of V rows) and fp32 (m, l)
            const int rr = (wave & 1) * PF_BM + (row - s.r0);  // the slot's row (head-major)
            const int64_t prow = (int64_t)item * 2 * PF_BM + rr;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) {
                const f32x4 x = ws.acc[mt][nt];
                st_dev64(a.part_o + (prow - rr) * PF_D + (mt * 2 * PF_BM + rr) * 16 + 4 * g,
                         (uint64_t)pack_bf16x2(x[0] * rl, x[1] * rl) |
                             ((uint64_t)pack_bf16x2(x[2] * rl, x[3] * rl) << 32));
            }
            if (g == 0)
                st_dev64(a.part_ml + prow * 2,
                         (uint64_t)__float_as_uint(l != 0.f ? -ws.nmb[nt] : -INFINITY) |
                             ((uint64_t)__float_as_uint(l) << 32));
        }
    }
    if (s.npieces == 1) {
        PF_STAMP(7);
        return;
    }
    merge_pieces(a, s, unit, item_base);
    PF_STAMP(7);
}

// Merge of a split (sub-block, kv head) pair, in the launch that computed its pieces. Piece p ran
// as item item_base + p * Hkv + hk and wrote its partial rows to that item's slot. The pair's
// (row, query head) outputs are cut into npieces shares, and the merge of share k (log-sum-exp
// in base 2, pieces in order) reads share k's rows of every piece's partial:
//  * each piece counts itself in at arrivals[item_base + hk] (its arrival index k), then waits
//    until all pieces have arrived, and merges share k; the last to arrive merges its share at
//    once. The wait ends early when no other piece has arrived for a.merge_stall_ticks (the
//    missing ones may not be resident yet, e.g. on a GPU shared with other work) and after
//    a.merge_wait_ticks in all (100 MHz real-time clock). The wait spreads the merge over the
//    pair's workgroups (one workgroup alone reads device-coherent data at a fraction of the
//    rate the pair's pieces reach together);
//  * each then adds (1 << 16) | (merged ? 1 << k : 0) to the pair's finish word
//    (arrivals[grid + item_base + hk]); the last to finish merges every share whose owner gave
//    up waiting (none, unless a piece ran long after the others) and resets both words to zero.
// Every wait ends; a piece that gives up costs time, not correctness. The pair's words sit at
// its first item: split items are numbered below the slot count and no other pair's first item
// is that one. The words must be zero on entry (the workspace contract). Should they not be,
// an arrival index k >= npieces takes no share and sets no bit, so every access stays inside
// the pair's rows; the pair's output is then not merged by this launch.
__device__ __forceinline__ void merge_pieces(const PrefillArgs& a, const SubBlock& s, int unit,
                                             int item_base) {
    const int np = s.npieces, nrows = s.r1 - s.r0;
    const PfUnit pu = pf_unit(a, unit);
    uint32_t* const arr = a.arrivals + item_base + unit;
    uint32_t* const fin = a.arrivals + a.grid + item_base + unit;
    __shared__ int s_k, s_go, s_missing;
    wait_stores();  // this wave's partial is written
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t k = __hip_atomic_fetch_add(arr, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        PF_STAMP(4);
        int go = k == (uint32_t)(np - 1);
        if (k < (uint32_t)(np - 1)) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            uint64_t t_seen = t0;
            uint32_t seen = k + 1;
            for (;;) {
                const uint32_t c =
                    __hip_atomic_load(arr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (c >= (uint32_t)np) {
                    go = 1;
                    break;
                }
                const uint64_t t = __builtin_amdgcn_s_memrealtime();
                if (c != seen) {
                    seen = c;
                    t_seen = t;
                }
                if (t - t0 > a.merge_wait_ticks || t - t_seen > a.merge_stall_ticks) break;
                __builtin_amdgcn_s_sleep(2);
            }
        }
        s_k = (int)min(k, (uint32_t)PF_MAXP);
        s_go = go;
        PF_STAMP(5);
    }
    __syncthreads();
    const int k = s_k;
    const bool go = s_go != 0;

    // 16 lanes per (row, query head), 8 channels each: a wave's load reads four consecutive slot
    // rows, 128 contiguous bytes in each of the 8 channel blocks. Group G of 16 lanes merges the
    // share's pairs G, G + GR, ...
    constexpr int GR = PF_THREADS / 16;
    const int G = threadIdx.x >> 4, c0 = 8 * (threadIdx.x & 15);
    const rsrc_t po = make_rsrc(a.part_o, (uint32_t)a.grid * PF_BM * 2 * PF_D * 2);
    const rsrc_t pml = make_rsrc(a.part_ml, (uint32_t)a.grid * PF_BM * 2 * 2 * 4);
    // piece p's partial slot; the pair q of the share (head-major: head q / nrows, row q % nrows)
    // is slot row rr = head * PF_BM + row
    auto slot_of = [&](int p) { return item_base + p * a.units + unit; };
    auto merge_share = [&](int share) {
        const int npairs = 2 * nrows;
        const int pb = share * npairs / np, pe = (share + 1) * npairs / np;
        constexpr int U = 2;  // pairs per group whose loads are in flight together
#pragma unroll 1
        for (int q0 = pb; q0 < pe; q0 += U * GR) {
            // (m, l) and the channels of every piece of U pairs in one round trip (an offset past
            // a buffer's range reads zeros without a memory access)
            u32x2 ml[U][PF_MAXP];
            u32x4 o[U][PF_MAXP];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int q = q0 + u * GR + G;
                const bool row_in = q < pe;
                const int hh = q >= nrows, rr = hh * PF_BM + q - hh * nrows;
#pragma unroll
                for (int p = 0; p < PF_MAXP; ++p) {
                    const bool in = row_in && p < np;
                    const int sl = slot_of(p);
                    ml[u][p] = __builtin_amdgcn_raw_buffer_load_b64(
                        pml, in ? (sl * 2 * PF_BM + rr) * 8 : -64, 0, CPOL_SC1);
                    // channels c0..c0 + 7: 16-channel block c0 / 16, half (c0 / 8) & 1
                    o[u][p] = __builtin_amdgcn_raw_buffer_load_b128(
                        po,
                        in ? (sl * 2 * PF_BM * PF_D + ((c0 >> 4) * 2 * PF_BM + rr) * 16 + (c0 & 8)) * 2
                           : -64,
                        0, CPOL_SC1);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int q = q0 + u * GR + G;
                if (q >= pe) continue;
                const int hh = q >= nrows, row = s.r0 + q - hh * nrows;
                float mx = -INFINITY;
#pragma unroll
                for (int p = 0; p < PF_MAXP; ++p)
                    mx = fmaxf(mx, p < np ? __uint_as_float(ml[u][p][0]) : -INFINITY);
                float num[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, den = 0.f;
#pragma unroll
                for (int p = 0; p < PF_MAXP; ++p) {
                    // piece weight: its softmax mass l * 2^(m - mx) (0 for a piece with no
                    // visible key)
                    const float m = __uint_as_float(ml[u][p][0]);
                    const float w =
                        p >= np || m == -INFINITY
                            ? 0.f
                            : __uint_as_float(ml[u][p][1]) * __builtin_amdgcn_exp2f(m - mx);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        num[2 * j] += bf16lo(o[u][p][j]) * w;
                        num[2 * j + 1] += bf16hi(o[u][p][j]) * w;
                    }
                    den += w;
                }
                const float rd = den != 0.f ? 1.f / den : 0.f;
                if (hh && !pu.has2) continue;  // an odd ratio's last pair has one head
                uint16_t* dst = a.out + row * a.o_st + (pu.qh0 + hh) * a.o_sh + c0;
                *reinterpret_cast<u32x4*>(dst) = u32x4{
                    pack_bf16x2(num[0] * rd, num[1] * rd), pack_bf16x2(num[2] * rd, num[3] * rd),
                    pack_bf16x2(num[4] * rd, num[5] * rd), pack_bf16x2(num[6] * rd, num[7] * rd)};
            }
        }
    };
    if (go) merge_share(k);  // go only when k < np
    PF_STAMP(6);
    if (threadIdx.x == 0) {
        const uint32_t mine = (1u << 16) | (go ? 1u << k : 0u);  // k < np <= PF_MAXP < 16
        const uint32_t old =
            __hip_atomic_fetch_add(fin, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int missing = -1;  // not the last to finish
        if ((int)(old >> 16) == np - 1) {
            missing = (int)(~(old | mine) & ((1u << np) - 1));
            __hip_atomic_store(arr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(fin, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_missing = missing;
    }
    __syncthreads();
    const int missing = s_missing;
    if (missing > 0)
        for (int share = 0; share < np; ++share)
            if ((missing >> share) & 1) merge_share(share);
}


// grid (max(slots, sub-blocks * Hkv)), block 256: workgroup w runs item w of the launch's item
// list (there are never more items than that), or nothing. A grid of one resident wave whose
// workgroups loop over items w, w + slots, ... measured slower (config 4 +28 %, long prefills
// +38 %): the dispatcher hands later workgroups to whichever CU frees up first, which balances
// uneven items better than a fixed assignment.
__global__ __launch_bounds__(PF_THREADS, IE_PREFILL_WG_PER_CU) void prefill_attention_kernel(
    PrefillArgs a) {
    // every wave reads the tile metadata and derives the workgroup's item itself
    __shared__ __attribute__((aligned(16))) PfLds lds;
    PF_STAMP(0);
    SubBlock s;
    int unit, kt_begin, kt_end, item_base;
    if (a.plan) {
        // the workgroup's row of the precomputed work list: one 64-byte load
        const int lane = threadIdx.x & 63;
        const int v = lane < PF_PLAN_FIELDS ? a.plan[PF_PLAN_FIELDS * blockIdx.x + lane] : 0;
        auto f = [&](int i) { return __builtin_amdgcn_readlane(v, i); };
        PF_STAMP(1);
        PF_STAMP_VALUE(8, f(0) ? f(4) : 0);
        if (!f(0)) return;
        unit = f(2);
        s.npieces = f(4);
        kt_begin = f(5);
        kt_end = f(6);
        s.npt = f(7);
        s.nct = f(8);
        s.ntiles = s.npt + s.nct;
        s.r0 = f(9);
        s.r1 = f(10);
        s.seq_start = f(11);
        s.P = f(12);
        s.slot = f(13);
        s.npp = 0;  // not read: the tile range comes with the row
        item_base = f(15);
    } else {
        Loc loc = schedule(a, blockIdx.x, reinterpret_cast<int*>(lds.k[1]));
        {
            int* f = reinterpret_cast<int*>(&loc);
#pragma unroll
            for (int i = 0; i < (int)(sizeof(Loc) / sizeof(int)); ++i) f[i] = uni(f[i]);
        }
        PF_STAMP(1);
        PF_STAMP_VALUE(8, loc.found ? loc.s.npieces : 0);
        if (!loc.found) return;
        s = loc.s;
        unit = loc.off % a.units;
        item_base = loc.item_base;
        piece_tiles(loc.s, loc.off / a.units, kt_begin, kt_end);
    }
    prefill_item(a, s, unit, kt_begin, kt_end, blockIdx.x, item_base, lds);
}

// grid (the prefill launch's grid), block 64: the launch's work list, as the main kernel's own
// schedule computes it, one row of PF_PLAN_FIELDS int32 per workgroup index w:
//   found, sub-block, unit, piece, pieces of the pair, first tile, end tile, prefix tiles,
//   chunk tiles, first row, end row, entry's first row, prefix length, cache slot,
//   straddling form, the pair's first item
// (tile kt < prefix tiles is prefix tile kt, else chunk tile kt - prefix tiles; rows of a
// workgroup with no item are zero). The main kernel runs from these rows when given them.
__global__ __launch_bounds__(IE_WAVE) void prefill_plan_kernel(PrefillArgs a, int32_t* rows) {
    __shared__ int tables[3 * PF_LDS_ENTRIES + 2];
    Loc loc = schedule(a, blockIdx.x, tables);
    {
        int* f = reinterpret_cast<int*>(&loc);
#pragma unroll
        for (int i = 0; i < (int)(sizeof(Loc) / sizeof(int)); ++i) f[i] = uni(f[i]);
    }
    if (threadIdx.x != 0) return;
    int32_t r[PF_PLAN_FIELDS] = {};
    if (loc.found) {
        const int hk = loc.off % a.units, piece = loc.off / a.units;
        int kb, ke;
        piece_tiles(loc.s, piece, kb, ke);
        const int v[16] = {1, loc.sb, hk, piece, loc.s.npieces, kb, ke, loc.s.npt, loc.s.nct,
                           loc.s.r0, loc.s.r1, loc.s.seq_start, loc.s.P, loc.s.slot,
                           loc.straddle, loc.item_base};
        for (int i = 0; i < PF_PLAN_FIELDS; ++i) r[i] = v[i];
    }
    for (int i = 0; i < PF_PLAN_FIELDS; ++i) rows[PF_PLAN_FIELDS * blockIdx.x + i] = r[i];
}

// How long a split piece waits for its pair's other pieces before leaving its share of the
// merge to the last one to finish, in ticks of the 100 MHz real-time clock: at most 100 us in
// all (IE_PREFILL_MERGE_WAIT_US) and at most 20 us without another piece arriving
// (IE_PREFILL_MERGE_STALL_US). Read at every call; a wait of 0 makes every piece but the last
// give up at once, which tests the fallback.
static uint64_t env_us_ticks(const char* name, long dflt) {
    const char* e = std::getenv(name);
    const long us = e && *e ? std::strtol(e, nullptr, 10) : dflt;
    return (uint64_t)std::max(0L, std::min(us, 10000000L)) * 100;
}

// Partial slots: one resident wave of main-kernel workgroups (split items never outnumber it).
static int prefill_slots() { return std::max(1, device_cu_count() * IE_PREFILL_WG_PER_CU); }

// Workspace: an arrival word and a finish word per partial slot (padded to 256 B; zero on entry,
// and every launch leaves them zero), then per partial slot PF_BM rows x 2 query heads of (m, l)
// fp32 and 128 bf16 channels. The layout depends on the device only, so one workspace serves
// every launch.
struct PrefillWs {
    size_t ml_off, o_off, bytes;
};
static PrefillWs prefill_ws(int slots) {
    PrefillWs w;
    w.ml_off = (2 * (size_t)slots * sizeof(uint32_t) + 255) / 256 * 256;
    w.o_off = w.ml_off + (size_t)slots * PF_BM * 2 * 2 * sizeof(float);
    w.bytes = w.o_off + (size_t)slots * PF_BM * 2 * PF_D * sizeof(uint16_t);
    return w;
}

}  // namespace ie

using namespace ie;

// The launch's grid: one resident wave of workgroups, or one workgroup per (sub-block, unit)
// pair when there are more (a unit is a KV head and one pair of its query heads).
static int64_t prefill_grid(int64_t nsb, int units) {
    return std::max<int64_t>(prefill_slots(), nsb * units);
}

// The schedule's part of the arguments (index arrays and sizes).
static hipError_t prefill_index_args(PrefillArgs& a, const int32_t* seq_ids,
                                     const int32_t* cu_seqlens, const int32_t* tile_start,
                                     int32_t num_tiles, int32_t block_m, int64_t num_tokens,
                                     int32_t num_q_heads, int32_t num_kv_heads,
                                     const int32_t* slot_ids, const int32_t* cu_cached,
                                     int32_t num_entries) {
    IE_REQUIRE(num_tokens >= 0 && num_tiles >= 0, "negative sizes");
    IE_REQUIRE(block_m > 0, "block_m must be positive");
    IE_REQUIRE(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0 &&
                   num_q_heads / num_kv_heads <= 16,
               "num_q_heads must be num_kv_heads times a GQA ratio of 1 to 16");
    IE_REQUIRE(num_entries >= 1, "num_entries (the length of slot_ids) must be at least 1");
    const int64_t nsb = (int64_t)num_tiles * ((block_m + PF_BM - 1) / PF_BM);
    IE_REQUIRE(nsb < (1 << 24), "too many tiles");
    IE_REQUIRE(num_tokens < ((int64_t)1 << 31), "too many tokens");
    a.seq_ids = seq_ids;
    a.cu_seqlens = cu_seqlens;
    a.tile_start = tile_start;
    a.slot_ids = slot_ids;
    a.cu_cached = cu_cached;
    a.block_m = block_m;
    a.sub_per_tile = (block_m + PF_BM - 1) / PF_BM;
    a.hq = num_q_heads;
    a.hkv = num_kv_heads;
    a.ratio = num_q_heads / num_kv_heads;
    a.npairs = (a.ratio + 1) / 2;
    a.units = num_kv_heads * a.npairs;
    a.nent = num_entries;
    a.ntok = (int)num_tokens;
    a.nsb = (int)nsb;
    a.grid = prefill_slots();
    return hipSuccess;
}

extern "C" size_t ie_prefill_attention_workspace_size(int32_t num_tiles, int32_t block_m,
                                                      int32_t num_kv_heads) {
    if (num_tiles <= 0 || block_m <= 0 || num_kv_heads <= 0) return 0;
    return prefill_ws(prefill_slots()).bytes;
}

extern "C" size_t ie_prefill_attention_workspace_counts_bytes(void) {
    return prefill_ws(prefill_slots()).ml_off;
}

// ie_prefill_attention and ie_prefill_attention_planned (plan: null, or the launch's work list).
static hipError_t prefill_launch(
    const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head, const ie_bf16* k,
    int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* v, int64_t v_stride_tok,
    int64_t v_stride_head, int64_t num_tokens, int32_t num_q_heads, const int32_t* seq_ids,
    const int32_t* cu_seqlens, const int32_t* tile_start, int32_t num_tiles, int32_t block_m,
    const ie_kv_cache* cache, const int32_t* slot_ids, const int32_t* cu_cached,
    int32_t num_entries, ie_bf16* out, int64_t out_stride_tok, int64_t out_stride_head,
    void* workspace, size_t workspace_bytes, const int32_t* plan, int64_t plan_rows,
    hipStream_t stream) {
    hipError_t e = check_cache(cache);
    if (e != hipSuccess) return e;
    PrefillArgs a{};
    e = prefill_index_args(a, seq_ids, cu_seqlens, tile_start, num_tiles, block_m, num_tokens,
                           num_q_heads, (int32_t)cache->num_kv_heads, slot_ids, cu_cached,
                           num_entries);
    if (e != hipSuccess) return e;
    if (num_tokens == 0 || num_tiles == 0) return hipSuccess;
    IE_REQUIRE(q && k && v && seq_ids && cu_seqlens && tile_start && slot_ids && cu_cached && out,
               "null pointer");
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    IE_REQUIRE(al16(q) && al16(k) && al16(v) && al16(out), "q/k/v/out must be 16-byte aligned");
    IE_REQUIRE(q_stride_tok % 8 == 0 && q_stride_head % 8 == 0 && k_stride_tok % 8 == 0 &&
                   k_stride_head % 8 == 0 && v_stride_tok % 8 == 0 && v_stride_head % 8 == 0 &&
                   out_stride_tok % 4 == 0 && out_stride_head % 4 == 0,
               "q/k/v/out rows must be 16-byte aligned with contiguous head_dim");
    // chunk rows are read through 32-bit buffer ranges whose end masks rows past the sub-block
    IE_REQUIRE(k_stride_tok >= PF_D && v_stride_tok >= PF_D,
               "k/v token stride must be at least head_dim elements");
    IE_REQUIRE(num_tokens * std::max(k_stride_tok, v_stride_tok) * 2 < ((int64_t)1 << 31),
               "k/v too large for 32-bit row offsets");
    IE_REQUIRE((reinterpret_cast<uintptr_t>(cache->k_calibration) & 15) == 0 &&
                   cache->cal_stride_head % 4 == 0 && cache->cal_stride_slot % 4 == 0,
               "k_calibration rows must be 16-byte aligned");
    const PrefillWs wsl = prefill_ws(a.grid);
    IE_REQUIRE(workspace != nullptr && workspace_bytes >= wsl.bytes && al16(workspace),
               "workspace too small");
    a.q = (const uint16_t*)q;
    a.q_st = q_stride_tok;
    a.q_sh = q_stride_head;
    a.k = (const uint16_t*)k;
    a.k_st = k_stride_tok;
    a.k_sh = k_stride_head;
    a.v = (const uint16_t*)v;
    a.v_st = v_stride_tok;
    a.v_sh = v_stride_head;
    a.c = *cache;
    a.out = (uint16_t*)out;
    a.o_st = out_stride_tok;
    a.o_sh = out_stride_head;
    a.arrivals = (uint32_t*)workspace;
    a.part_ml = (float*)((char*)workspace + wsl.ml_off);
    a.part_o = (uint16_t*)((char*)workspace + wsl.o_off);
    a.qk_scale = (float)(0.08838834764831845 * 1.4426950408889634);  // D^-0.5 * log2(e), D = 128
    a.merge_wait_ticks = env_us_ticks("IE_PREFILL_MERGE_WAIT_US", 100);
    a.merge_stall_ticks = env_us_ticks("IE_PREFILL_MERGE_STALL_US", 20);
    const int64_t grid = prefill_grid(a.nsb, a.units);
    if (plan) {
        IE_REQUIRE(plan_rows >= grid && (reinterpret_cast<uintptr_t>(plan) & 3) == 0,
                   "plan must hold ie_prefill_attention_grid(...) rows of 16 int32");
        a.plan = plan;
    }
    hipLaunchKernelGGL(prefill_attention_kernel, dim3((unsigned)grid), dim3(PF_THREADS), 0, stream,
                       a);
    return hipGetLastError();
}

extern "C" hipError_t ie_prefill_attention(
    const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head, const ie_bf16* k,
    int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* v, int64_t v_stride_tok,
    int64_t v_stride_head, int64_t num_tokens, int32_t num_q_heads, const int32_t* seq_ids,
    const int32_t* cu_seqlens, const int32_t* tile_start, int32_t num_tiles, int32_t block_m,
    const ie_kv_cache* cache, const int32_t* slot_ids, const int32_t* cu_cached,
    int32_t num_entries, ie_bf16* out,
    int64_t out_stride_tok, int64_t out_stride_head, void* workspace, size_t workspace_bytes,
    hipStream_t stream) {
    return prefill_launch(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, v,
                          v_stride_tok, v_stride_head, num_tokens, num_q_heads, seq_ids,
                          cu_seqlens, tile_start, num_tiles, block_m, cache, slot_ids, cu_cached,
                          num_entries, out, out_stride_tok, out_stride_head, workspace,
                          workspace_bytes, nullptr, 0, stream);
}

extern "C" hipError_t ie_prefill_attention_planned(
    const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head, const ie_bf16* k,
    int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* v, int64_t v_stride_tok,
    int64_t v_stride_head, int64_t num_tokens, int32_t num_q_heads, const int32_t* seq_ids,
    const int32_t* cu_seqlens, const int32_t* tile_start, int32_t num_tiles, int32_t block_m,
    const ie_kv_cache* cache, const int32_t* slot_ids, const int32_t* cu_cached,
    int32_t num_entries, const int32_t* plan, int64_t plan_rows, ie_bf16* out,
    int64_t out_stride_tok, int64_t out_stride_head, void* workspace, size_t workspace_bytes,
    hipStream_t stream) {
    IE_REQUIRE(plan != nullptr, "null plan");
    return prefill_launch(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, v,
                          v_stride_tok, v_stride_head, num_tokens, num_q_heads, seq_ids,
                          cu_seqlens, tile_start, num_tiles, block_m, cache, slot_ids, cu_cached,
                          num_entries, out, out_stride_tok, out_stride_head, workspace,
                          workspace_bytes, plan, plan_rows, stream);
}

extern "C" int32_t ie_prefill_attention_grid(int32_t num_tiles, int32_t block_m,
                                             int32_t num_q_heads, int32_t num_kv_heads) {
    if (num_tiles <= 0 || block_m <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 ||
        num_q_heads % num_kv_heads != 0)
        return 0;
    const int64_t nsb = (int64_t)num_tiles * ((block_m + PF_BM - 1) / PF_BM);
    const int units = num_kv_heads * ((num_q_heads / num_kv_heads + 1) / 2);
    return (int32_t)std::min<int64_t>(prefill_grid(nsb, units), INT32_MAX);
}

extern "C" hipError_t ie_prefill_attention_plan(const int32_t* seq_ids, const int32_t* cu_seqlens,
                                                const int32_t* tile_start, int32_t num_tiles,
                                                int32_t block_m, int64_t num_tokens,
                                                int32_t num_q_heads, int32_t num_kv_heads,
                                                const int32_t* slot_ids,
                                                const int32_t* cu_cached, int32_t num_entries,
                                                int32_t* rows, hipStream_t stream) {
    PrefillArgs a{};
    hipError_t e = prefill_index_args(a, seq_ids, cu_seqlens, tile_start, num_tiles, block_m,
                                      num_tokens, num_q_heads, num_kv_heads, slot_ids, cu_cached,
                                      num_entries);
    if (e != hipSuccess) return e;
    if (num_tiles == 0) return hipSuccess;
    IE_REQUIRE(seq_ids && cu_seqlens && tile_start && slot_ids && cu_cached && rows,
               "null pointer");
    const unsigned grid = (unsigned)prefill_grid(a.nsb, a.units);
    hipLaunchKernelGGL(prefill_plan_kernel, dim3(grid), dim3(IE_WAVE), 0, stream, a, rows);
    return hipGetLastError();
}

#ifdef IE_PREFILL_PHASE_STAMPS
// Diagnostic build only: copies the first `count` words of the phase-stamp array to host memory
// (clear: then zeroes the array).
extern "C" hipError_t ie_prefill_phase_stamps_copy(unsigned long long* host, size_t count,
                                                   int clear) {
    IE_REQUIRE(count <= (size_t)PF_STAMP_WGS * 9, "count beyond the stamp array");
    hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(ie::pf_phase_stamps),
                                       count * sizeof(unsigned long long));
    if (e != hipSuccess || !clear) return e;
    static unsigned long long zeros[PF_STAMP_WGS * 9];
    return hipMemcpyToSymbol(HIP_SYMBOL(ie::pf_phase_stamps), zeros, sizeof(zeros));
}
#endif
