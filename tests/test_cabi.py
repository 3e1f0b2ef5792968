"""The C ABI library loads, exports everything include/ie_attn.h declares, and rejects bad
arguments on the host before touching a device (CPU only: no compute calls)."""

import ctypes

import pytest
import torch

HIP_ERROR_INVALID_VALUE = 1


def test_library_exports_every_declared_symbol(native):
    lib = native.cabi()
    names = native.header_functions()
    assert len(names) >= 11
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert lib.ie_attn_version() >> 16 == 1


def test_torch_ops_registered(ie):
    ops = ie.kernels.ops()
    for name in ["quantize_kv_prefill", "fused_rope_kv_decode", "fused_norm_rope_prefill",
                 "decode_attention", "decode_attention_rope", "dequantize_kv_prefix",
                 "prefill_attention", "decode_attention_workspace_size", "sample", "add_rms_norm",
                 "silu_mul", "skinny_matmul", "skinny_matmul_silu_mul", "skinny_matmul_norm",
                 "skinny_matmul_residual_", "prefill_plan", "decode_plan", "rope_tables",
                 "skinny_weight_swizzle", "decode_step_prologue", "lm_head_greedy"]:
        assert hasattr(ops, name), name


def test_null_cache_rejected_on_host(native):
    lib = native.cabi()
    fn = lib.ie_decode_attention
    fn.restype = ctypes.c_int
    null = ctypes.c_void_p(0)
    rc = fn(null, ctypes.c_int64(128), ctypes.c_int64(128), ctypes.c_int32(1), ctypes.c_int32(16),
            null, null, null, null, ctypes.c_float(0.1), null, ctypes.c_int64(2048),
            ctypes.c_int64(128), null, ctypes.c_size_t(0), null)
    assert rc == HIP_ERROR_INVALID_VALUE
    assert b"null" in lib.ie_attn_last_error()


def test_bad_geometry_rejected_on_host(native):
    lib = native.cabi()
    desc = native.KVCacheDesc(16, 16, 16, 16, 16, 2, 8, 64, 64, 8 * 64 * 64, 64 * 64, 64,
                              8 * 64, 64, 8 * 64, 64)  # head_dim 64: unsupported
    fn = lib.ie_quantize_kv_prefill
    fn.restype = ctypes.c_int
    null = ctypes.c_void_p(0)
    rc = fn(null, ctypes.c_int64(0), ctypes.c_int64(0), null, ctypes.c_int64(0),
            ctypes.c_int64(0), ctypes.c_int64(0), null, null, null, null, ctypes.c_int32(1),
            ctypes.byref(desc), null)
    assert rc == HIP_ERROR_INVALID_VALUE
    assert b"head_dim" in lib.ie_attn_last_error()


def test_workspace_size_formula(native):
    """The arrival counts (one uint32 per sequence and query head, room for at least 1024
    sequences of 128 heads, padded to 256 bytes), then one fp32 partial (128 outputs, m, l) per
    query head and work entry; the work entries are the launch's grid: the target, or target + B
    above it."""
    lib = native.cabi()
    t_max = lib.ie_decode_attention_max_splits(8)
    assert t_max >= 1
    lib.ie_decode_attention_grid.restype = ctypes.c_int32
    prev = 0
    for B in (1, 64, 65, 96, 128, 129, 256, 257, 300, 1024):
        # the target grows with the batch (8-, 4- then 2-wave workgroups) and holds it while
        # any launch shape can
        target = lib.ie_decode_attention_target(ctypes.c_int32(B), ctypes.c_int32(8))
        assert prev <= target <= t_max and (B <= target or target == t_max)
        prev = target
        grid = lib.ie_decode_attention_grid(ctypes.c_int32(B), ctypes.c_int32(8))
        assert grid == (target if B <= target else target + B)
        # counts: one per sequence and query head (the most any GQA ratio uses), for at least
        # 1024 sequences and 128 heads; partials: one per query head and work entry of the
        # largest grid (cdiv(Hq, 2) units: GQA 2)
        counts = -(-(max(B, 1024) * 128) * 4 // 256) * 256
        assert lib.ie_decode_attention_workspace_size(B, 16, 128) == counts + 16 * grid * 130 * 4


def test_ops_refuse_cpu_tensors(ie):
    c = ie.make_layer_cache(2, 8, 64, 128, device="cpu")
    q = torch.zeros(1, 16, 128, dtype=torch.bfloat16)
    i = torch.zeros(1, dtype=torch.int32)
    with pytest.raises((RuntimeError, NotImplementedError)):
        ie.decode_attention(q, c, i, i, i, 0.1)


def test_decode_attention_rope_null_k_rejected_on_host(native):
    """The fused decode entry point checks its own arguments (here a null k) after the decode
    ones, on the host, before any launch."""
    lib = native.cabi()
    desc = native.KVCacheDesc(256, 256, 256, 256, 256, 2, 8, 64, 128, 8 * 64 * 128, 64 * 128, 128,
                              8 * 64, 64, 8 * 128, 128)
    fn = lib.ie_decode_attention_rope
    fn.restype = ctypes.c_int
    p, null, i64 = ctypes.c_void_p(256), ctypes.c_void_p(0), ctypes.c_int64
    ws = lib.ie_decode_attention_workspace_size(1, 16, 128)
    rc = fn(p, i64(4096), i64(128), null, i64(4096), i64(128), p, i64(4096), i64(128), p, p,
            p, i64(64), p, i64(64), ctypes.c_float(1e-6), ctypes.c_int32(1), ctypes.c_int32(16),
            ctypes.byref(desc), p, p, p, ctypes.c_float(0.1), p, i64(2048), i64(128), p,
            ctypes.c_size_t(ws), null)
    assert rc == HIP_ERROR_INVALID_VALUE
    assert b"null" in lib.ie_attn_last_error()


def test_quantize_too_many_tokens_rejected_on_host(native):
    lib = native.cabi()
    # a well-formed descriptor (head_dim 128) over fake aligned addresses: rejected before launch
    desc = native.KVCacheDesc(256, 256, 256, 256, 256, 2, 8, 64, 128, 8 * 64 * 128, 64 * 128, 128,
                              8 * 64, 64, 8 * 128, 128)
    fn = lib.ie_quantize_kv_prefill
    fn.restype = ctypes.c_int
    p = ctypes.c_void_p(256)
    rc = fn(p, ctypes.c_int64(1024), ctypes.c_int64(128), p, ctypes.c_int64(1024),
            ctypes.c_int64(128), ctypes.c_int64(65535 * 32), p, p, p, p, ctypes.c_int32(2),
            ctypes.byref(desc), ctypes.c_void_p(0))
    assert rc == HIP_ERROR_INVALID_VALUE
    assert b"too many tokens" in lib.ie_attn_last_error()


def test_workspace_count_regions_and_prefill_grid(native):
    """The bytes a caller clears to reset a workspace: the decode arrival counts (max(B, 1024)
    * max(Hq, 128) uint32, padded to 256 bytes: the offset of the partials in the size formula
    above, the same for every call of up to 1024 sequences and 128 heads) and
    the prefill arrival and finish words (two per resident workgroup, padded to 256 bytes, within
    the prefill workspace). The prefill launch's grid: one resident wave of workgroups or one
    workgroup per (128-row sub-block, KV head), whichever is more."""
    lib = native.cabi()
    for B in (1, 64, 1024, 1025, 3000):
        for hq in (16, 32, 2, 256):
            want = -(-(max(B, 1024) * max(hq, 128) * 4) // 256) * 256
            assert lib.ie_decode_attention_workspace_counts_bytes(B, hq) == want
    lib.ie_prefill_attention_workspace_size.restype = ctypes.c_size_t
    ws = lib.ie_prefill_attention_workspace_size(ctypes.c_int32(8), ctypes.c_int32(128),
                                                 ctypes.c_int32(8))
    cb = lib.ie_prefill_attention_workspace_counts_bytes()
    slots = lib.ie_prefill_attention_grid(1, 128, 16, 8)  # one sub-block: the resident wave
    assert cb == -(-(2 * slots * 4) // 256) * 256 and 0 < cb < ws
    for tiles, bm in ((1, 128), (64, 128), (300, 128), (300, 192), (1000, 16)):
        nsb = tiles * -(-bm // 128)
        # one workgroup per (sub-block, KV head x query-head pair) when they outnumber the slots
        for hq, hkv in ((16, 8), (32, 8), (40, 8), (8, 8), (2, 1)):
            units = hkv * ((hq // hkv + 1) // 2)
            assert lib.ie_prefill_attention_grid(tiles, bm, hq, hkv) == max(slots, nsb * units)
    assert lib.ie_prefill_attention_grid(4, 128, 12, 8) == 0  # not a multiple: no launch


def test_prefill_plan_rejects_bad_sizes_on_host(native):
    lib = native.cabi()
    fn = lib.ie_prefill_attention_plan
    fn.restype = ctypes.c_int
    p, null = ctypes.c_void_p(256), ctypes.c_void_p(0)
    i32 = ctypes.c_int32
    rc = fn(p, p, p, i32(4), i32(0), ctypes.c_int64(100), i32(16), i32(8), p, p, i32(3), p, null)
    assert rc == HIP_ERROR_INVALID_VALUE and b"block_m" in lib.ie_attn_last_error()
    rc = fn(p, p, p, i32(4), i32(128), ctypes.c_int64(100), i32(16), i32(8), p, p, i32(0), p, null)
    assert rc == HIP_ERROR_INVALID_VALUE and b"num_entries" in lib.ie_attn_last_error()
    for hq, hkv in ((12, 8), (136, 8)):  # not a multiple; a ratio above 16
        rc = fn(p, p, p, i32(4), i32(128), ctypes.c_int64(100), i32(hq), i32(hkv), p, p, i32(3),
                p, null)
        assert rc == HIP_ERROR_INVALID_VALUE and b"GQA ratio" in lib.ie_attn_last_error()


def test_prefill_planned_rejects_bad_plans_on_host(native):
    """ie_prefill_attention_planned: a null plan, and a plan with fewer rows than the launch's
    grid, are refused before any launch (the pointers here are never dereferenced)."""
    lib = native.cabi()
    fn = lib.ie_prefill_attention_planned
    fn.restype = ctypes.c_int
    lib.ie_prefill_attention_workspace_size.restype = ctypes.c_size_t
    i32, i64 = ctypes.c_int32, ctypes.c_int64
    p = ctypes.c_void_p(1 << 20)  # aligned stand-in address
    desc = native.KVCacheDesc(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 4, 8, 1024, 128,
                              8 * 1024 * 128, 1024 * 128, 128, 8 * 1024, 1024, 8 * 128, 128)
    tiles, bm, hq, hkv = 8, 128, 16, 8
    grid = lib.ie_prefill_attention_grid(tiles, bm, hq, hkv)
    ws = lib.ie_prefill_attention_workspace_size(i32(tiles), i32(bm), i32(hkv))

    def call(plan, rows):
        return fn(p, i64(2048), i64(128), p, i64(1024), i64(128), p, i64(1024), i64(128),
                  i64(1024), i32(hq), p, p, p, i32(tiles), i32(bm), ctypes.byref(desc), p, p,
                  i32(3), plan, i64(rows), p, i64(2048), i64(128), p, ctypes.c_size_t(ws),
                  ctypes.c_void_p(0))

    assert call(ctypes.c_void_p(0), grid) == HIP_ERROR_INVALID_VALUE
    assert b"null plan" in lib.ie_attn_last_error()
    assert call(p, grid - 1) == HIP_ERROR_INVALID_VALUE
    assert b"plan must hold" in lib.ie_attn_last_error()


def test_skinny_gemm_fused_rejects_bad_flags_on_host(native):
    """ie_skinny_gemm_fused: an undefined flag combination, a negative or infinite eps with
    IE_SKINNY_NORM, the gate/up form with n_tiles 4, a swizzled weight with 8-row tiles, 3 tiles
    outside the swizzled gate/up form and the fragment-order flags outside the forms that take
    them are refused before any launch (the pointers here are never dereferenced)."""
    lib = native.cabi()
    fn = lib.ie_skinny_gemm_fused
    fn.restype = ctypes.c_int
    i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    p = ctypes.c_void_p(1 << 20)

    def call(flags, eps=1e-6, n_tiles=1):
        return fn(p, i64(2048), i32(32), p, i64(2048), i32(4096), i32(2048), i32(n_tiles),
                  i32(flags), f32(eps), p, i64(4096), ctypes.c_void_p(0))

    for flags in (64, 1 | 4, 2 | 4, 7, 8 | 1 | 4, -1):
        assert call(flags) == HIP_ERROR_INVALID_VALUE, flags
        assert b"flags" in lib.ie_attn_last_error()
    for flags in (8, 8 | 1, 8 | 4):  # a swizzled weight: no 8-row tiles
        assert call(flags, n_tiles=0) == HIP_ERROR_INVALID_VALUE, flags
        assert b"swizzled" in lib.ie_attn_last_error()
    for eps in (-1.0, float("inf"), float("nan")):
        assert call(1, eps) == HIP_ERROR_INVALID_VALUE, eps
        assert b"eps" in lib.ie_attn_last_error()
    assert call(2, n_tiles=4) == HIP_ERROR_INVALID_VALUE
    assert b"n_tiles" in lib.ie_attn_last_error()
    for flags in (0, 2, 8, 8 | 1):  # 3 tiles: only the swizzled gate/up form
        assert call(flags, n_tiles=3) == HIP_ERROR_INVALID_VALUE, flags
        assert b"n_tiles" in lib.ie_attn_last_error()
    assert call(8 | 2, n_tiles=5) == HIP_ERROR_INVALID_VALUE  # paired gate/up: 1 ... 4
    assert b"n_tiles" in lib.ie_attn_last_error()
    for flags in (32, 32 | 2, 32 | 8, 32 | 1 | 8):  # y in fragment order: swizzled gate/up only
        assert call(flags) == HIP_ERROR_INVALID_VALUE, flags
        assert b"fragment" in lib.ie_attn_last_error()
    for flags in (16 | 1, 16 | 2, 16 | 8 | 2):  # x in fragment order: plain or residual only
        assert call(flags) == HIP_ERROR_INVALID_VALUE, flags
        assert b"fragment" in lib.ie_attn_last_error()


def test_decode_planned_rejects_bad_plans_on_host(native):
    """ie_decode_attention_planned / ie_decode_attention_rope_planned: a null plan, fewer rows
    than the launch's work entries, and a misaligned plan are refused before any launch (the
    pointers here are never dereferenced)."""
    lib = native.cabi()
    lib.ie_decode_attention_workspace_size.restype = ctypes.c_size_t
    i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    p = ctypes.c_void_p(1 << 20)
    desc = native.KVCacheDesc(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 4, 8, 1024, 128,
                              8 * 1024 * 128, 1024 * 128, 128, 8 * 1024, 1024, 8 * 128, 128)
    B, hq = 3, 16
    ws = lib.ie_decode_attention_workspace_size(i32(B), i32(hq), i32(128))
    grid = lib.ie_decode_attention_grid(i32(B), i32(8))
    assert grid > 0
    plain = lib.ie_decode_attention_planned
    plain.restype = ctypes.c_int
    rope = lib.ie_decode_attention_rope_planned
    rope.restype = ctypes.c_int

    def call_plain(plan, rows):
        return plain(p, i64(2048), i64(128), i32(B), i32(hq), ctypes.byref(desc), p, p, p, plan,
                     i64(rows), f32(0.1), p, i64(2048), i64(128), p, ctypes.c_size_t(ws),
                     ctypes.c_void_p(0))

    def call_rope(plan, rows):
        return rope(p, i64(4096), i64(128), p, i64(4096), i64(128), p, i64(4096), i64(128), p,
                    p, p, i64(64), p, i64(64), f32(1e-6), i32(B), i32(hq), ctypes.byref(desc),
                    p, p, p, plan, i64(rows), f32(0.1), p, i64(2048), i64(128), p,
                    ctypes.c_size_t(ws), ctypes.c_void_p(0))

    for call in (call_plain, call_rope):
        assert call(ctypes.c_void_p(0), grid) == HIP_ERROR_INVALID_VALUE
        assert b"null plan" in lib.ie_attn_last_error()
        assert call(p, grid - 1) == HIP_ERROR_INVALID_VALUE
        assert b"plan must hold" in lib.ie_attn_last_error()
        assert call(ctypes.c_void_p((1 << 20) + 4), grid) == HIP_ERROR_INVALID_VALUE
        assert b"aligned" in lib.ie_attn_last_error()


def test_lm_head_greedy_and_prologue_reject_bad_arguments_on_host(native):
    """ie_skinny_lm_head_greedy: flags other than 0 / NORM, k other than 2048, a null tokens
    pointer and a short workspace; ie_decode_step_prologue: a model_dim that is not a multiple
    of 8 and a null embedding: refused before any launch (the pointers are never dereferenced)."""
    lib = native.cabi()
    i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    p = ctypes.c_void_p(1 << 20)
    null = ctypes.c_void_p(0)
    lib.ie_skinny_lm_head_greedy_workspace_size.restype = ctypes.c_size_t
    wsb = lib.ie_skinny_lm_head_greedy_workspace_size()
    assert wsb >= 64 * 8 + 4
    fn = lib.ie_skinny_lm_head_greedy
    fn.restype = ctypes.c_int

    def greedy(flags=1, k=2048, tokens=p, ws_bytes=wsb):
        return fn(p, i64(k), i32(32), p, i32(81920), i32(k), i32(2), i32(flags), f32(1e-6), p,
                  i64(81920), tokens, i64(1), p, p, ctypes.c_size_t(ws_bytes), null)

    for kw, msg in ((dict(flags=2), b"flags"), (dict(k=1024), b"2048"),
                    (dict(tokens=null), b"null"), (dict(ws_bytes=wsb - 8), b"workspace")):
        assert greedy(**kw) == HIP_ERROR_INVALID_VALUE, kw
        assert msg in lib.ie_attn_last_error(), kw
    pro = lib.ie_decode_step_prologue
    pro.restype = ctypes.c_int

    def prologue(dim=2048, embed=p):
        return pro(p, p, i32(32), i32(8), p, p, i32(64), p, p, p, embed, i64(2048), i64(1000),
                   i32(dim), p, i64(2048), null)

    assert prologue(dim=100) == HIP_ERROR_INVALID_VALUE
    assert b"multiple of 8" in lib.ie_attn_last_error()
    assert prologue(embed=null) == HIP_ERROR_INVALID_VALUE
    assert b"null" in lib.ie_attn_last_error()
