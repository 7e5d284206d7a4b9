"""Offline CPU quantizers that produce the packed operands (numpy / torch CPU).

These play the role of the reference's converters (roblennon/mac-kernels-public
bench/wan_int8_convert.py, bench/qwen_int8_convert.py): they run once, on the host, to build the
packed weights the GPU kernels consume.  They are input generators, not the product's compute
path.

GGUF: simple absmax/min-max block quantizers writing the standard block layouts
(docs/research/2026-10-03-gguf-on-metal.md:18-36).  They are not ggml's search-based
quantizers; bit-exactness is judged on the decode of the same bytes, not on quantizer equality.
"""
from __future__ import annotations

import numpy as np

from .gguf import GGUF_TYPES, gguf_type_id, GGUF_NAMES

# ggml IQ4_NL levels (public ggml kvalues_iq4nl).
IQ4NL_LEVELS = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int8)

def _f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def _f16_bytes(x):
    return _f16(x).view(np.uint8).reshape(*np.shape(x), 2)


def _safe_div(a, b):
    b = np.where(b == 0, 1.0, b)
    return a / b


def _signed_absmax(x, axis=-1):
    """Value of largest magnitude (with its sign) along axis."""
    idx = np.abs(x).argmax(axis=axis)
    return np.take_along_axis(x, np.expand_dims(idx, axis), axis=axis).squeeze(axis)


def _pack_nibbles_32(q):
    """q [..., 32] in 0..15 -> 16 bytes: byte j = q[j] | q[j+16] << 4."""
    return (q[..., :16] | (q[..., 16:] << 4)).astype(np.uint8)


def _q4_k_scales(sc, mn):
    """Pack eight 6-bit (scale, min) pairs into the 12-byte K-quant layout."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint8)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 0xF) | ((mn[..., 4:8] & 0xF) << 4)
    return out


def quantize_gguf(w, qtype):
    """fp32 [N, K] -> uint8 [N, K/qk*ts] in the GGUF block layout of `qtype`."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    name = GGUF_NAMES[gguf_type_id(qtype)]
    _, qk, ts = GGUF_TYPES[name]
    n, k = w.shape
    assert k % qk == 0, f"K={k} is not a multiple of the {qk}-value block"
    nb = n * k // qk
    x = w.reshape(nb, qk)
    out = np.zeros((nb, ts), dtype=np.uint8)
    if name in ("Q8_0",):
        d = np.abs(x).max(-1) / 127.0
        d16 = _f16(d).astype(np.float32)
        q = np.clip(np.rint(_safe_div(x, d16[:, None])), -127, 127).astype(np.int8)
        out[:, 0:2] = _f16_bytes(d)
        out[:, 2:34] = q.view(np.uint8)
    elif name in ("Q4_0", "Q5_0"):
        lv = 8 if name == "Q4_0" else 16
        d = _signed_absmax(x) / -lv
        d16 = _f16(d).astype(np.float32)
        q = np.clip(np.rint(_safe_div(x, d16[:, None])) + lv, 0, 2 * lv - 1).astype(np.uint32)
        out[:, 0:2] = _f16_bytes(d)
        if name == "Q4_0":
            out[:, 2:18] = _pack_nibbles_32(q)
        else:
            qh = ((q >> 4) & 1) << np.arange(32, dtype=np.uint32)
            out[:, 2:6] = qh.sum(-1).astype(np.uint32).view(np.uint8).reshape(nb, 4)
            out[:, 6:22] = _pack_nibbles_32(q & 0xF)
    elif name in ("Q4_1", "Q5_1"):
        lv = 15 if name == "Q4_1" else 31
        mn, mx = x.min(-1), x.max(-1)
        d = (mx - mn) / lv
        d16 = _f16(d).astype(np.float32)
        m16 = _f16(mn).astype(np.float32)
        q = np.clip(np.rint(_safe_div(x - m16[:, None], d16[:, None])), 0, lv).astype(np.uint32)
        out[:, 0:2] = _f16_bytes(d)
        out[:, 2:4] = _f16_bytes(mn)
        if name == "Q4_1":
            out[:, 4:20] = _pack_nibbles_32(q)
        else:
            qh = ((q >> 4) & 1) << np.arange(32, dtype=np.uint32)
            out[:, 4:8] = qh.sum(-1).astype(np.uint32).view(np.uint8).reshape(nb, 4)
            out[:, 8:24] = _pack_nibbles_32(q & 0xF)
    elif name == "IQ4_NL":
        lev = IQ4NL_LEVELS.astype(np.float32)
        d = _signed_absmax(x) / -127.0
        d16 = _f16(d).astype(np.float32)
        t = _safe_div(x, d16[:, None])
        q = np.abs(t[..., None] - lev).argmin(-1).astype(np.uint32)
        out[:, 0:2] = _f16_bytes(d)
        out[:, 2:18] = _pack_nibbles_32(q)
    elif name in ("Q4_K", "Q5_K"):
        lv = 15 if name == "Q4_K" else 31
        s = x.reshape(nb, 8, 32)
        mnv = np.minimum(s.min(-1), 0.0)
        scale = (s.max(-1) - mnv) / lv
        mins = -mnv
        d = scale.max(-1) / 63.0
        dmin = mins.max(-1) / 63.0
        d16, dm16 = _f16(d).astype(np.float32), _f16(dmin).astype(np.float32)
        sc = np.clip(np.rint(_safe_div(scale, d16[:, None])), 0, 63)
        mc = np.clip(np.rint(_safe_div(mins, dm16[:, None])), 0, 63)
        eff_d = d16[:, None] * sc
        eff_m = dm16[:, None] * mc
        q = np.clip(np.rint(_safe_div(s + eff_m[..., None], eff_d[..., None])), 0, lv).astype(np.uint32)
        out[:, 0:2] = _f16_bytes(d)
        out[:, 2:4] = _f16_bytes(dmin)
        out[:, 4:16] = _q4_k_scales(sc, mc)
        lo = (q & 0xF).reshape(nb, 4, 2, 32)
        qs = (lo[:, :, 0, :] | (lo[:, :, 1, :] << 4)).reshape(nb, 128).astype(np.uint8)
        if name == "Q4_K":
            out[:, 16:144] = qs
        else:
            hb = ((q >> 4) & 1).reshape(nb, 8, 32)
            qh = (hb << np.arange(8, dtype=np.uint32)[None, :, None]).sum(1).astype(np.uint8)
            out[:, 16:48] = qh
            out[:, 48:176] = qs
    elif name == "Q6_K":
        s = x.reshape(nb, 16, 16)
        sub = _signed_absmax(s) / -32.0
        d = np.abs(sub).max(-1) / 127.0
        d16 = _f16(d).astype(np.float32)
        sc = np.clip(np.rint(_safe_div(sub, d16[:, None])), -128, 127)
        eff = d16[:, None] * sc
        q = (np.clip(np.rint(_safe_div(s, eff[..., None])), -32, 31) + 32).astype(np.uint32).reshape(nb, 256)
        ql = np.zeros((nb, 128), dtype=np.uint32)
        qh = np.zeros((nb, 64), dtype=np.uint32)
        for v in range(256):
            h, r = v >> 7, v & 127
            ql[:, 64 * h + (r & 63)] |= (q[:, v] & 0xF) << (4 * (r >> 6))
            qh[:, 32 * h + (r & 31)] |= ((q[:, v] >> 4) & 3) << (2 * (r >> 5))
        out[:, 0:128] = ql.astype(np.uint8)
        out[:, 128:192] = qh.astype(np.uint8)
        out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
        out[:, 208:210] = _f16_bytes(d)
    elif name == "Q3_K":
        s = x.reshape(nb, 16, 16)
        sub = _signed_absmax(s) / -4.0
        d = np.abs(sub).max(-1) / 31.0
        d16 = _f16(d).astype(np.float32)
        s6 = np.clip(np.rint(_safe_div(sub, d16[:, None])), -32, 31)
        eff = d16[:, None] * s6
        q = np.clip(np.rint(_safe_div(s, eff[..., None])), -4, 3).astype(np.int32).reshape(nb, 256)
        hbit = (q >= 0).astype(np.uint32)
        low = (q + 4 * (1 - hbit)).astype(np.uint32)  # 0..3
        qs = np.zeros((nb, 64), dtype=np.uint32)
        hm = np.zeros((nb, 32), dtype=np.uint32)
        for v in range(256):
            h, t2, i = v >> 7, (v >> 5) & 3, v & 31
            qs[:, 32 * h + i] |= low[:, v] << (2 * t2)
            hm[:, i] |= hbit[:, v] << (v >> 5)
        sc = (s6 + 32).astype(np.uint32)  # 0..63
        scb = np.zeros((nb, 12), dtype=np.uint32)
        for j in range(16):
            scb[:, j & 7] |= (sc[:, j] & 0xF) << (4 * (j >> 3))
            scb[:, 8 + (j & 3)] |= ((sc[:, j] >> 4) & 3) << (2 * (j >> 2))
        out[:, 0:32] = hm.astype(np.uint8)
        out[:, 32:96] = qs.astype(np.uint8)
        out[:, 96:108] = scb.astype(np.uint8)
        out[:, 108:110] = _f16_bytes(d)
    elif name == "Q2_K":
        s = x.reshape(nb, 16, 16)
        mnv = np.minimum(s.min(-1), 0.0)
        scale = (s.max(-1) - mnv) / 3.0
        mins = -mnv
        d = scale.max(-1) / 15.0
        dmin = mins.max(-1) / 15.0
        d16, dm16 = _f16(d).astype(np.float32), _f16(dmin).astype(np.float32)
        sc = np.clip(np.rint(_safe_div(scale, d16[:, None])), 0, 15)
        mc = np.clip(np.rint(_safe_div(mins, dm16[:, None])), 0, 15)
        eff_d = d16[:, None] * sc
        eff_m = dm16[:, None] * mc
        q = np.clip(np.rint(_safe_div(s + eff_m[..., None], eff_d[..., None])), 0, 3).astype(np.uint32).reshape(nb, 256)
        qs = np.zeros((nb, 64), dtype=np.uint32)
        for v in range(256):
            h, t2, i = v >> 7, (v >> 5) & 3, v & 31
            qs[:, 32 * h + i] |= q[:, v] << (2 * t2)
        out[:, 0:16] = (sc.astype(np.uint32) | (mc.astype(np.uint32) << 4)).astype(np.uint8)
        out[:, 16:80] = qs.astype(np.uint8)
        out[:, 80:82] = _f16_bytes(d)
        out[:, 82:84] = _f16_bytes(dmin)
    elif name == "IQ4_XS":
        lev = IQ4NL_LEVELS.astype(np.float32)
        s = x.reshape(nb, 8, 32)
        sub = _signed_absmax(s) / -127.0
        d = np.abs(sub).max(-1) / 32.0
        d16 = _f16(d).astype(np.float32)
        ls = np.clip(np.rint(_safe_div(sub, d16[:, None])) + 32, 0, 63).astype(np.uint32)
        dl = d16[:, None] * (ls.astype(np.float32) - 32)
        t = _safe_div(s, dl[..., None])
        q = np.abs(t[..., None] - lev).argmin(-1).astype(np.uint32)  # nb, 8, 32
        sh = np.zeros(nb, dtype=np.uint32)
        for j in range(8):
            sh |= ((ls[:, j] >> 4) & 3) << (2 * j)
        sl = np.zeros((nb, 4), dtype=np.uint32)
        for j in range(8):
            sl[:, j >> 1] |= (ls[:, j] & 0xF) << (4 * (j & 1))
        out[:, 0:2] = _f16_bytes(d)
        out[:, 2:4] = sh.astype(np.uint16).view(np.uint8).reshape(nb, 2)
        out[:, 4:8] = sl.astype(np.uint8)
        out[:, 8:136] = (q[..., :16] | (q[..., 16:] << 4)).reshape(nb, 128).astype(np.uint8)
    else:  # pragma: no cover
        raise ValueError(name)
    return out.reshape(n, k // qk * ts)


# ------------------------------------------------------------------------------------------------
# ConvRot rotation and INT8 (modal/weight_error_app.py:90-127)
# ------------------------------------------------------------------------------------------------

def hadamard_signs(g: int) -> np.ndarray:
    """Unnormalized +-1 block Hadamard of size g: the Kronecker power of
    H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] for g = 4^p (weight_error_app.py:90-98), with
    an H2 = [[1,1],[1,-1]] factor as the most significant digit for g = 2 * 4^p."""
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    p, rest = 0, g
    while rest % 4 == 0 and rest > 1:
        rest //= 4
        p += 1
    if rest not in (1, 2) or g < 2:
        raise ValueError(f"Hadamard size must be 4^p or 2*4^p, got {g}")
    h = np.array([[1.0]]) if rest == 1 else np.array([[1.0, 1.0], [1.0, -1.0]])
    for _ in range(p):
        h = np.kron(h, h4)
    return h


def rotate(w: np.ndarray, g: int) -> np.ndarray:
    """Per-group rotation w[:, grp] @ H^T (H normalized, symmetric), computed in float64 and rounded
    once to float32."""
    w = np.asarray(w)
    if not g:
        return w.astype(np.float32)
    n, k = w.shape
    assert k % g == 0, f"K={k} is not a multiple of the rotation group {g}"
    h = hadamard_signs(g) / np.sqrt(g)
    return (w.astype(np.float64).reshape(n, k // g, g) @ h.T).reshape(n, k).astype(np.float32)


def quantize_int8_rowwise(w: np.ndarray):
    """Per-row symmetric int8 (weight_error_app.py:109-115): scale = max(absmax/127, 1e-30) in fp32,
    q = clamp(rne(w / scale), -128, 127)."""
    w = np.asarray(w, dtype=np.float32)
    scale = np.maximum(np.abs(w).max(axis=1, keepdims=True) / np.float32(127.0), np.float32(1e-30)).astype(np.float32)
    q = np.clip(np.rint(w / scale), -128, 127).astype(np.int8)
    return q, scale.reshape(-1)


def quantize_int8_convrot_weight(w: np.ndarray, convrot_groupsize: int = 256):
    """ConvRot INT8 weight: rotate by the block Hadamard along K, then per-row int8.
    Returns (q int8 [N, K] in the rotated basis, scale fp32 [N])."""
    return quantize_int8_rowwise(rotate(w, convrot_groupsize))


# ------------------------------------------------------------------------------------------------
# W4A8 / W6A8 (AsymW4A8Int8 storage; modal/weight_error_app.py:132-323)
# ------------------------------------------------------------------------------------------------

# Fixed 16-level Lloyd-Max table for near-Gaussian groups (modal/weight_error_app.py:132-135).
FIXED_CODEBOOK = np.array([
    -0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
    0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671], dtype=np.float32)
KURTOSIS_GATE = -0.1      # excess kurtosis at or below which the fixed table is used
KURTOSIS_SAMPLE = 1 << 19
ALS_ITERS = 2
ROW_BUDGET = 1 << 22       # elements per row block / codebook row sample


def _torch():
    import torch
    return torch


def _nearest(values, table):
    """Index of the nearest entry of an ascending table (ties go to the lower index)."""
    torch = _torch()
    last = table.numel() - 1
    pos = torch.searchsorted(table, values.contiguous())
    lo = (pos - 1).clamp(0, last)
    hi = pos.clamp(0, last)
    return torch.where((values - table[hi]).abs() < (values - table[lo]).abs(), hi, lo)


def _nearest_rows(values, tables):
    """Row-wise nearest: values [R, G], tables [R, L] ascending per row."""
    torch = _torch()
    last = tables.shape[-1] - 1
    pos = torch.searchsorted(tables.contiguous(), values.contiguous())
    lo = (pos - 1).clamp(0, last)
    hi = pos.clamp(0, last)
    dlo = (values - torch.gather(tables, 1, lo)).abs()
    dhi = (values - torch.gather(tables, 1, hi)).abs()
    return torch.where(dhi < dlo, hi, lo)


def fit_codebook(samples, levels=16, iterations=25, sample_size=300000):
    """Quantile-initialized 1-D k-means over normalized weights."""
    torch = _torch()
    s = samples.flatten()
    if s.numel() > sample_size:
        gen = torch.Generator().manual_seed(0)
        s = s[torch.randint(0, s.numel(), (sample_size,), generator=gen)]
    s = s.float()
    cb = torch.quantile(s, torch.linspace(0, 1, levels))
    for _ in range(iterations):
        idx = (s.unsqueeze(-1) - cb).abs().argmin(-1)
        new = cb.clone()
        for i in range(levels):
            sel = idx == i
            if sel.any():
                new[i] = s[sel].mean()
        cb = new
    return cb.contiguous()


def choose_codebook(normalized):
    """Fixed table when the normalized groups are light-tailed (excess kurtosis <= -0.1), else fitted."""
    torch = _torch()
    v = normalized.detach().flatten()
    if v.numel() > KURTOSIS_SAMPLE:
        gen = torch.Generator().manual_seed(0)
        v = v[torch.randint(0, v.numel(), (KURTOSIS_SAMPLE,), generator=gen)]
    v = v.float()
    kurt = ((v - v.mean()) / (v.std() + 1e-9)).pow(4).mean() - 3.0
    if kurt.item() <= KURTOSIS_GATE:
        return torch.from_numpy(FIXED_CODEBOOK.copy())
    return fit_codebook(normalized)


def _grid(table, s_rel_f32):
    return (table.view(1, 1, -1) * s_rel_f32.unsqueeze(-1)).round_().clamp_(-127, 127)


def _assign_grid(target, levels):
    n, groups, gs = target.shape
    idx = _nearest_rows(target.reshape(n * groups, gs), levels.reshape(n * groups, -1).contiguous())
    return idx.reshape(n, groups, gs)


def _neighbour_scales(s_rel):
    """The stored scale one unit in the last place below and above (e4m3 raw bits, or fp16 bits)."""
    torch = _torch()
    if s_rel.dtype == torch.float8_e4m3fn:
        raw = s_rel.view(torch.uint8).to(torch.int16)
        dn = (raw - 1).clamp(min=1).to(torch.uint8).view(torch.float8_e4m3fn)
        up = (raw + 1).clamp(max=0x7E).to(torch.uint8).view(torch.float8_e4m3fn)
    else:
        raw = s_rel.view(torch.int16).to(torch.int32)
        dn = (raw - 1).clamp(min=1).to(torch.int16).view(torch.float16)
        up = (raw + 1).clamp(max=0x7BFF).to(torch.int16).view(torch.float16)
    return dn, up


def _quantize_block(rot, group_size, bits, table, uniform, s_rel_dtype):
    torch = _torch()
    n, k = rot.shape
    groups = k // group_size
    g = rot.float().view(n, groups, group_size)
    amax = g.abs().amax(-1, keepdim=True)
    if uniform:
        L = (1 << (bits - 1)) - 1
        gscale = (amax / L).clamp(min=1e-8)

        def assign(t):
            return (t.round().clamp(-L, L) + L).to(torch.int64)
    else:
        gscale = amax.clamp(min=1e-8)

        def assign(t):
            return _nearest(t, table)
    idx = assign(g / gscale)
    for _ in range(ALS_ITERS):
        lq = table[idx]
        gscale = ((g * lq).sum(-1, keepdim=True) / (lq * lq).sum(-1, keepdim=True).clamp(min=1e-8)).clamp(min=1e-8)
        idx = assign(g / gscale)
    shifted = table[idx] * gscale
    s_channel = (shifted.abs().amax(dim=(1, 2)) / 127.0).clamp(min=1e-8)
    s_rel = (gscale.squeeze(-1) / s_channel.unsqueeze(1)).float().to(s_rel_dtype)
    target = g / s_channel.view(-1, 1, 1)
    if uniform:
        best_s = s_rel
        levels = _grid(table, s_rel.float())
        best_idx = _assign_grid(target, levels)
        best_err = (torch.gather(levels, 2, best_idx) - target).pow(2).sum(-1)
        for cand in _neighbour_scales(s_rel):
            levels = _grid(table, cand.float())
            ci = _assign_grid(target, levels)
            err = (torch.gather(levels, 2, ci) - target).pow(2).sum(-1)
            better = err < best_err
            best_err = torch.where(better, err, best_err)
            best_s = torch.where(better, cand.float(), best_s.float()).to(s_rel_dtype)
            best_idx = torch.where(better.unsqueeze(-1), ci, best_idx)
        s_rel = best_s
        codes = best_idx + ((1 << (bits - 1)) - ((1 << (bits - 1)) - 1))
    else:
        codes = _assign_grid(target, _grid(table, s_rel.float()))
    return codes.reshape(n, k), s_rel.contiguous(), s_channel.float().contiguous()


def pack_codes(codes, bits):
    """codes [N, K] -> int8 [N, K*bits/8]: nibble plane (byte j = c[2j] | c[2j+1] << 4), then for
    6 bits the 2-bit plane (byte j = sum_i ((c[4j+i] >> 4) & 3) << 2i)."""
    torch = _torch()
    c = codes.to(torch.int32)
    low = (c[:, 0::2] & 0xF) | ((c[:, 1::2] & 0xF) << 4)
    if bits == 4:
        return low.to(torch.uint8).view(torch.int8).contiguous()
    hi = torch.zeros_like(c[:, 0::4])
    for j in range(4):
        hi |= ((c[:, j::4] >> 4) & 3) << (2 * j)
    return torch.cat([low, hi], 1).to(torch.uint8).view(torch.int8).contiguous()


def quantize_w4a8_int8_weight(w, bits=4, group_size=16, convrot_groupsize=256, codebook="auto",
                              s_rel_dtype=None):
    """AsymW4A8Int8 packing of an [N, K] weight.

    bits=4, codebook="auto": the reference's default (fixed or fitted 16-level codebook);
    codebook=None: uniform symmetric levels (+-(2^(bits-1)-1)) with the +-1 ulp scale search the
    reference applies to 6 bits; bits=6 always uses uniform levels.  s_rel_dtype defaults to
    float8_e4m3fn (torch.float16 is accepted).
    Returns (qdata int8 [N, K*bits/8], s_rel [N, K/group_size], s_channel fp32 [N], codebook or None),
    with qdata in the ConvRot-rotated basis.
    """
    torch = _torch()
    s_rel_dtype = s_rel_dtype or torch.float8_e4m3fn
    w = torch.as_tensor(np.asarray(w, dtype=np.float32))
    n, k = w.shape
    assert bits in (4, 6) and k % group_size == 0 and (not convrot_groupsize or k % convrot_groupsize == 0)
    uniform = bits == 6 or codebook is None
    if uniform:
        L = (1 << (bits - 1)) - 1
        table = torch.arange(-L, L + 1, dtype=torch.float32)
        cb_out = None
    elif isinstance(codebook, str):
        max_rows = max(1, ROW_BUDGET // max(k, 1))
        sample = w if n <= max_rows else w.index_select(0, torch.linspace(0, n - 1, max_rows).long())
        rs = torch.from_numpy(rotate(sample.numpy(), convrot_groupsize))
        grouped = rs.view(sample.shape[0], k // group_size, group_size)
        table = choose_codebook(grouped / grouped.abs().amax(-1, keepdim=True).clamp(min=1e-8))
        cb_out = table
    else:
        table = torch.as_tensor(codebook, dtype=torch.float32)
        cb_out = table
    block = max(1, ROW_BUDGET // max(k, 1))
    parts = []
    for r0 in range(0, n, block):
        rot = torch.from_numpy(rotate(w[r0:r0 + block].numpy(), convrot_groupsize))
        parts.append(_quantize_block(rot, group_size, bits, table, uniform, s_rel_dtype))
    codes = torch.cat([p[0] for p in parts], 0)
    s_rel = torch.cat([p[1] for p in parts], 0)
    s_ch = torch.cat([p[2] for p in parts], 0)
    return pack_codes(codes, bits), s_rel, s_ch, cb_out
