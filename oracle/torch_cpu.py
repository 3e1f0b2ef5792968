"""PyTorch-on-CPU restatement of the reference's attention math, for the benchmark's CPU
baseline (test infrastructure only; see oracle/__init__.py). It runs on the host cores with
torch's own threading, fp32 throughout (dequant, scores, softmax, PV), batches streamed in
slices of at most 16 sequences to bound memory.

decode_attention      qwen3-1.7b/kernels.py:73-264: softmax(scale * k_scale * <q, k_int8>) over
                      tokens [0, cached_len + 1), weights times v_scale * v_int8.
quantize_kv_prefill   qwen3-1.7b/kernels.py:717-865: first-chunk calibration, x / cal, per-row
                      scale max(amax, 1e-6) / 127, round half to even, clamp to +-127.
prefill_attention     qwen3-1.7b/kernels.py:987-1126 fed by dequantize_kv_prefix (:868-932):
                      each packed row attends to its entry's dequantized prefix and causally to
                      its own chunk.

Pinned by tests/test_oracle_torch_cpu.py against the numpy oracle and its float64 forms.
"""

import torch

SLICE = 16


def decode_attention(q, k_cache, v_cache, k_scale, v_scale, cached_lens, slot_ids, num_decoding,
                     scale):
    """q fp32/bf16 [B, Hq, D] (CPU); cache tensors on the CPU. Returns fp32 [nd, Hq, D].
    As the reference kernel arranges it (kernels.py:175-186): scores = <q, k_int8> times the
    token's k_scale * scale, and PV weights p * v_scale against v_int8, per sequence on its
    contiguous cache rows (a slice of sequences at a time)."""
    nd = int(num_decoding)
    B, hq, D = q.shape
    hkv = k_cache.shape[1]
    g = hq // hkv
    out = torch.empty(nd, hq, D, dtype=torch.float32)
    for b0 in range(0, nd, SLICE):
        for b in range(b0, min(nd, b0 + SLICE)):
            n, slot = int(cached_lens[b]) + 1, int(slot_ids[b])
            k = k_cache[slot, :, :n].float()  # [Hkv, n, D]
            v = v_cache[slot, :, :n].float()
            qs = q[b].float().view(hkv, g, D)
            s = torch.matmul(qs, k.transpose(-1, -2)) * (k_scale[slot, :, None, :n] * scale)
            p = torch.softmax(s, dim=-1) * v_scale[slot, :, None, :n]
            out[b] = torch.matmul(p, v).view(hq, D)
    return out


def quantize_kv_prefill(k, v, cu_seqlens, slot_ids, cached_lens, num_decoding, k_cache, v_cache,
                        k_scale, v_scale, k_calibration):
    """In-place prefill write into CPU cache tensors. k, v [N, Hkv, D] (bf16 or fp32)."""
    S = len(cu_seqlens) - 1
    for b in range(int(num_decoding), S):
        start, end = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        if end == start:
            continue
        slot, c0 = int(slot_ids[b]), int(cached_lens[b])
        kc = k[start:end].float().transpose(0, 1)  # [Hkv, L, D]
        vc = v[start:end].float().transpose(0, 1)
        if c0 == 0:
            k_calibration[slot, :, 0] = kc.abs().amax(dim=1).clamp_min(1e-3)
        x = kc / k_calibration[slot, :, 0][:, None, :]
        for src, qd, sd in ((x, k_cache, k_scale), (vc, v_cache, v_scale)):
            s = src.abs().amax(dim=-1).clamp_min(1e-6) / 127.0
            qd[slot, :, c0:c0 + end - start] = torch.round(src / s[..., None]).clamp_(
                -127, 127).to(torch.int8)
            sd[slot, :, c0:c0 + end - start] = s


def prefill_attention(q, k, v, cu_seqlens, slot_ids, cu_cached, num_decoding, k_cache, v_cache,
                      k_scale, v_scale, k_calibration):
    """Rows of every prefilling entry (index >= num_decoding); q [N, Hq, D], k/v [N, Hkv, D].
    Returns fp32 [N, Hq, D] with only those rows written (others zero)."""
    N, hq, D = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = torch.zeros(N, hq, D, dtype=torch.float32)
    for e in range(int(num_decoding), len(cu_seqlens) - 1):
        s0, s1 = int(cu_seqlens[e]), int(cu_seqlens[e + 1])
        L = s1 - s0
        if L == 0:
            continue
        P = int(cu_cached[e + 1]) - int(cu_cached[e])
        slot = int(slot_ids[e])
        kp = (k_cache[slot, :, :P].float() * k_scale[slot, :, :P, None]) * k_calibration[slot]
        vp = v_cache[slot, :, :P].float() * v_scale[slot, :, :P, None]
        kk = torch.cat([kp, k[s0:s1].float().transpose(0, 1)], dim=1)  # [Hkv, P + L, D]
        vv = torch.cat([vp, v[s0:s1].float().transpose(0, 1)], dim=1)
        qs = q[s0:s1].float().view(L, hkv, g, D).permute(1, 2, 0, 3)  # [Hkv, g, L, D]
        s = torch.matmul(qs, kk[:, None].transpose(-1, -2)) * D ** -0.5  # [Hkv, g, L, P + L]
        key = torch.arange(P + L)
        row = torch.arange(L)[:, None]
        s.masked_fill_(key[None, :] > P + row, float("-inf"))
        p = torch.softmax(s, dim=-1)
        o = torch.matmul(p, vv[:, None])  # [Hkv, g, L, D]
        out[s0:s1] = o.permute(2, 0, 1, 3).reshape(L, hq, D)
    return out
