"""GPU parity of the attention core (hydra_attn_fwd) against the CPU oracle
(SDPA restatement of attention.py:268-327, itself pinned to an fp64 brute
force).  bf16 runs on the MFMA kernel, fp32/fp16 and odd head dims on the
generic kernel.  Inputs are bf16-representable so both sides see identical
values; the oracle runs in fp32.  Tolerance: 2e-2 (bf16), 1e-5 (fp32)."""
from __future__ import annotations

import math

import pytest
import torch

from conftest import max_rel_err
from oracle import ccgqa as occ

pytestmark = pytest.mark.gpu


def _qkv(B, Hq, Hkv, S, hd, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).float()
    return mk(B, Hq, S, hd), mk(B, Hkv, S, hd), mk(B, Hkv, S, hd)


CASES = [
    # B, Hq, Hkv, S, hd
    (4, 4, 1, 512, 64),
    (2, 8, 2, 512, 16),
    (1, 4, 4, 257, 32),
    (2, 8, 1, 100, 128),
    (1, 2, 2, 1, 64),
    (1, 4, 2, 31, 64),
    (3, 6, 3, 65, 16),
    (2, 28, 4, 520, 16),  # config 5's heads: groups of 7, head_dim 16
]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_attention_bf16_mfma(cuda, case, causal):
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    B, Hq, Hkv, S, hd = case
    q, k, v = _qkv(*case, seed=sum(case))
    out, lse = attention_forward(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)),
                                 causal=causal, want_lse=True)
    ref = occ.attention(q, k, v, causal=causal)
    assert max_rel_err(out.cpu(), ref) < 2e-2
    # LSE: log sum_t exp(scale * q.k_t) over visible keys
    G = Hq // Hkv
    kk = k.repeat_interleave(G, 1)
    logits = (q @ kk.transpose(-1, -2)) / math.sqrt(hd)
    if causal:
        logits = logits.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    ref_lse = torch.logsumexp(logits, -1)
    assert (lse.cpu() - ref_lse).abs().max().item() < 2e-2


@pytest.mark.parametrize("generic", [False, True])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("case", [(2, 8, 2, 512, 16), (1, 4, 1, 77, 64), (1, 2, 1, 19, 6),
                                  (2, 4, 2, 130, 8), (1, 2, 1, 70, 128), (1, 3, 3, 33, 32)])
def test_attention_valu(cuda, monkeypatch, dtype, case, causal, generic):
    """The VALU kernels (fp32 / fp16): the key-split kernel (head_dim 8..128)
    and the one-thread-per-row kernel (odd head dims, or forced), output and
    LSE."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    if generic:
        monkeypatch.setenv("HYDRA_ATTN_GENERIC", "1")
    B, Hq, Hkv, S, hd = case
    q, k, v = _qkv(*case, seed=3)
    out, lse = attention_forward(*(t.to(cuda, dtype) for t in (q, k, v)), causal=causal, want_lse=True)
    ref = occ.attention(q, k, v, causal=causal)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert max_rel_err(out.cpu(), ref) < tol
    kk = k.repeat_interleave(Hq // Hkv, 1)
    logits = (q.double() @ kk.double().transpose(-1, -2)) / math.sqrt(hd)
    if causal:
        logits = logits.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    assert (lse.cpu().double() - torch.logsumexp(logits, -1)).abs().max().item() < 10 * tol


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attention_reference_mask_mode(cuda, dtype):
    """mask_mode REFERENCE_SDPA reproduces attention.py:268-299 literally."""
    from hydra_amd.attention.backends.ccgqa.ops import MASK_REFERENCE_SDPA, attention_forward

    B, Hq, Hkv, S, hd = 2, 4, 2, 70, 32
    q, k, v = _qkv(B, Hq, Hkv, S, hd, seed=11)
    g = torch.Generator().manual_seed(12)
    mask = (torch.rand(B, S, generator=g) > 0.2).long()
    mask[:, 0] = 1
    out, _ = attention_forward(*(t.to(cuda, dtype) for t in (q, k, v)), causal=True,
                               key_mask=mask.to(cuda), mask_mode=MASK_REFERENCE_SDPA)
    ref = occ.attention(q, k, v, causal=True, mask=mask)
    assert max_rel_err(out.cpu(), ref) < (1e-5 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attention_key_padding_mode(cuda, dtype):
    from hydra_amd.attention.backends.ccgqa.ops import MASK_KEY_PADDING, attention_forward

    B, Hq, Hkv, S, hd = 2, 4, 1, 90, 64
    q, k, v = _qkv(B, Hq, Hkv, S, hd, seed=13)
    g = torch.Generator().manual_seed(14)
    mask = (torch.rand(B, S, generator=g) > 0.3).long()
    mask[:, 0] = 1
    out, _ = attention_forward(*(t.to(cuda, dtype) for t in (q, k, v)), causal=True,
                               key_mask=mask.to(cuda), mask_mode=MASK_KEY_PADDING)
    ref = occ.attention_key_padding(q, k, v, causal=True, mask=mask)
    assert max_rel_err(out.cpu(), ref) < (1e-5 if dtype == torch.float32 else 2e-2)


def test_attention_fully_masked_row_is_zero(cuda):
    from hydra_amd.attention.backends.ccgqa.ops import MASK_KEY_PADDING, attention_forward

    q, k, v = _qkv(1, 2, 1, 40, 64, seed=15)
    mask = torch.ones(1, 40, dtype=torch.long)
    mask[0, :5] = 0  # queries 0..4 see no key
    out, lse = attention_forward(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), causal=True,
                                 key_mask=mask.to(cuda), mask_mode=MASK_KEY_PADDING, want_lse=True)
    assert torch.count_nonzero(out[:, :, :5].cpu()) == 0
    assert torch.isinf(lse[:, :, :5].cpu()).all()
    assert torch.isfinite(out.cpu()).all()


def test_attention_c3_full_size(cuda):
    """Config 3 core at full size: B4, Hq4/Hkv1, S4096, hd64, causal."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    q, k, v = _qkv(4, 4, 1, 4096, 64, seed=21)
    out, _ = attention_forward(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), causal=True)
    ref = occ.attention(q, k, v, causal=True)
    assert max_rel_err(out.cpu(), ref) < 2e-2


def test_attention_merged_output_layout(cuda):
    """Writing straight into a [B,S,Hq,hd] buffer equals the transposed copy."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    B, Hq, Hkv, S, hd = 2, 4, 1, 130, 64
    q, k, v = (t.to(cuda, torch.bfloat16) for t in _qkv(B, Hq, Hkv, S, hd, seed=22))
    o1, _ = attention_forward(q, k, v, causal=True)
    buf = torch.empty(B, S, Hq, hd, dtype=torch.bfloat16, device=cuda)
    attention_forward(q, k, v, causal=True, out=buf.transpose(1, 2))
    assert torch.equal(buf.transpose(1, 2).cpu(), o1.cpu())


def test_ccgqa_attention_fused_api(cuda):
    from hydra_amd.attention.backends.ccgqa.kernels import ccgqa_attention_fused

    q, k, v = _qkv(2, 4, 2, 96, 32, seed=23)
    out = ccgqa_attention_fused(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), is_causal=True)
    assert max_rel_err(out.cpu(), occ.attention(q, k, v, causal=True)) < 2e-2


def test_attention_deterministic(cuda):
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    q, k, v = (t.to(cuda, torch.bfloat16) for t in _qkv(2, 4, 1, 300, 64, seed=24))
    a, _ = attention_forward(q, k, v, causal=True)
    b, _ = attention_forward(q, k, v, causal=True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("sched", [None, "streamk"])
@pytest.mark.parametrize("case", [(4, 4, 1, 512, 64), (2, 8, 2, 256, 16), (1, 4, 4, 136, 32), (1, 2, 1, 64, 128)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_v_transposed_layout(cuda, monkeypatch, case, causal, sched):
    """V handed over as [B,Hkv,hd,S] (keys contiguous): the bf16 kernel stages
    it without a transpose.  Under the stream-K schedule the result equals
    the row-major V path bit for bit (same kernel, same order); the default
    key-split schedule folds the keys in another order, within bf16
    rounding of it."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    if sched:
        monkeypatch.setenv("HYDRA_ATTN_SCHED", sched)
    B, Hq, Hkv, S, hd = case
    q, k, v = _qkv(*case, seed=31)
    qd, kd = q.to(cuda, torch.bfloat16), k.to(cuda, torch.bfloat16)
    vt = v.transpose(2, 3).contiguous().to(cuda, torch.bfloat16)  # [B,Hkv,hd,S]
    out_t, _ = attention_forward(qd, kd, vt.transpose(2, 3), causal=causal)
    out_r, _ = attention_forward(qd, kd, v.to(cuda, torch.bfloat16), causal=causal)
    assert max_rel_err(out_t.cpu(), occ.attention(q, k, v, causal=causal)) < 2e-2
    if sched == "streamk":
        assert torch.equal(out_t.cpu(), out_r.cpu())
    else:
        assert max_rel_err(out_t.cpu(), out_r.float().cpu()) < 2e-2


def test_attention_v_transposed_odd_length_generic(cuda):
    """S not a multiple of 8 with transposed V goes to the generic kernel."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    q, k, v = _qkv(1, 4, 1, 37, 64, seed=32)
    vt = v.transpose(2, 3).contiguous().to(cuda, torch.bfloat16)
    out, _ = attention_forward(q.to(cuda, torch.bfloat16), k.to(cuda, torch.bfloat16),
                               vt.transpose(2, 3), causal=True)
    assert max_rel_err(out.cpu(), occ.attention(q, k, v, causal=True)) < 2e-2


SPLIT_CASES = [
    # B, Hq, Hkv, S, hd, causal, mask mode
    ((2, 8, 2, 512, 16), True, "none"),
    ((1, 4, 1, 1000, 64), True, "key_padding"),
    ((2, 4, 4, 300, 32), False, "none"),
    ((1, 8, 1, 257, 128), True, "none"),
    ((2, 4, 2, 200, 64), True, "reference"),
    ((1, 2, 1, 700, 64), False, "key_padding"),
]


@pytest.mark.parametrize("wgs", ["0", "3", "7", "64", "509"])
@pytest.mark.parametrize("case", SPLIT_CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}" for c in SPLIT_CASES])
def test_attention_split_chunks(cuda, monkeypatch, case, wgs):
    """The bf16 kernel shares the key tiles of all items equally among
    `wgs` workgroups (stream-K), so items are cut at arbitrary tiles and
    merged by a second kernel; wgs=0 runs one workgroup per item.  Every
    schedule gives the oracle's result, the LSE of the unsplit run (one
    workgroup), and identical bits on a repeated call."""
    from hydra_amd.attention.backends.ccgqa.ops import (MASK_KEY_PADDING, MASK_NONE,
                                                        MASK_REFERENCE_SDPA, attention_forward)

    (B, Hq, Hkv, S, hd), causal, mode = case
    q, k, v = _qkv(B, Hq, Hkv, S, hd, seed=S + hd)
    mask = None
    mm = {"none": MASK_NONE, "key_padding": MASK_KEY_PADDING, "reference": MASK_REFERENCE_SDPA}[mode]
    if mode != "none":
        g = torch.Generator().manual_seed(S)
        mask = (torch.rand(B, S, generator=g) > 0.25).long()
        mask[:, 0] = 1
        mask[0, 1:70] = 0  # a run of padding longer than one tile
    dev = lambda t: t.to(cuda, torch.bfloat16)
    kw = dict(causal=causal, key_mask=None if mask is None else mask.to(cuda), mask_mode=mm, want_lse=True)
    monkeypatch.setenv("HYDRA_ATTN_WGS", "1")  # one range: no item is split
    whole, whole_lse = attention_forward(dev(q), dev(k), dev(v), **kw)
    monkeypatch.setenv("HYDRA_ATTN_WGS", wgs)
    out, lse = attention_forward(dev(q), dev(k), dev(v), **kw)
    out2, lse2 = attention_forward(dev(q), dev(k), dev(v), **kw)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    if mode == "key_padding":
        ref = occ.attention_key_padding(q, k, v, causal=causal, mask=mask)
    else:
        ref = occ.attention(q, k, v, causal=causal, mask=mask)
    assert max_rel_err(out.cpu(), ref) < 2e-2
    assert max_rel_err(whole.cpu(), ref) < 2e-2
    assert max_rel_err(out.cpu(), whole.float().cpu()) < 2e-2
    fin = torch.isfinite(whole_lse)
    assert torch.equal(fin, torch.isfinite(lse))
    # P is rounded to bf16 against a per-chunk running max, so the row sums
    # agree to the bf16 rounding bound: |d log l| <= 2^-8.
    assert (lse[fin] - whole_lse[fin]).abs().max().item() < 2 ** -8


def test_attention_split_fully_masked_rows(cuda, monkeypatch):
    """Rows that see no key in any chunk come out as zeros with LSE -inf."""
    from hydra_amd.attention.backends.ccgqa.ops import MASK_KEY_PADDING, attention_forward

    monkeypatch.setenv("HYDRA_ATTN_WGS", "5")
    q, k, v = _qkv(1, 4, 1, 400, 64, seed=16)
    mask = torch.ones(1, 400, dtype=torch.long)
    mask[0, :150] = 0  # queries 0..149 see no key; later rows span several chunks
    out, lse = attention_forward(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), causal=True,
                                 key_mask=mask.to(cuda), mask_mode=MASK_KEY_PADDING, want_lse=True)
    assert torch.count_nonzero(out[:, :, :150].cpu()) == 0
    assert torch.isinf(lse[:, :, :150].cpu()).all()
    ref = occ.attention_key_padding(q, k, v, causal=True, mask=mask)
    assert max_rel_err(out[:, :, 150:].cpu(), ref[:, :, 150:]) < 2e-2


def _normed_qkv(B, Hq, Hkv, S, hd, temp, seed):
    """q of unit norm and k of norm |temp| per row (CCGQAAttention's QK-norm),
    bf16-representable, as the prep kernel hands them to attention."""
    g = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(B, Hq, S, hd, generator=g), dim=-1).to(torch.bfloat16).float()
    k = (nrm(torch.randn(B, Hkv, S, hd, generator=g), dim=-1) * temp).to(torch.bfloat16).float()
    v = torch.randn(B, Hkv, S, hd, generator=g).to(torch.bfloat16).float()
    return q, k, v


FIXED_CASES = [
    # B, Hq, Hkv, S, hd, temperature, causal
    (4, 4, 1, 512, 64, 1.0, True),
    (2, 8, 2, 300, 16, 4.0, True),
    (1, 4, 4, 257, 32, 5.66, False),
    (2, 8, 1, 100, 128, 11.3, True),
    (1, 2, 1, 64, 64, -8.0, False),
    (1, 4, 1, 2048, 64, 40.0, True),
    (2, 28, 4, 300, 16, 4.0, True),  # config 5's heads, temperature sqrt(16)
]


@pytest.mark.parametrize("wgs", [None, "7"])
@pytest.mark.parametrize("case", FIXED_CASES, ids=[str(c) for c in FIXED_CASES])
def test_attention_fixed_reference_max(cuda, monkeypatch, case, wgs):
    """Given a bound on |q.k| (QK-norm: 1.03 |temperature|), the bf16 kernel
    takes the fixed reference max instead of a running row max: the output
    matches the oracle and the online-max kernel, the LSE matches the
    closed form, also when stream-K cuts the items into chunks."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward, qk_norm_score_bound

    B, Hq, Hkv, S, hd, temp, causal = case
    if wgs is not None:
        monkeypatch.setenv("HYDRA_ATTN_WGS", wgs)
    q, k, v = _normed_qkv(B, Hq, Hkv, S, hd, temp, seed=S + hd)
    dev = lambda t: t.to(cuda, torch.bfloat16)
    beta = qk_norm_score_bound(temp)
    out_f, lse_f = attention_forward(dev(q), dev(k), dev(v), causal=causal, want_lse=True,
                                     score_bound=beta)
    out_o, lse_o = attention_forward(dev(q), dev(k), dev(v), causal=causal, want_lse=True)
    ref = occ.attention(q, k, v, causal=causal)
    assert max_rel_err(out_f.cpu(), ref) < 2e-2
    assert max_rel_err(out_f.cpu(), out_o.float().cpu()) < 2e-2
    G = Hq // Hkv
    logits = (q @ k.repeat_interleave(G, 1).transpose(-1, -2)) / math.sqrt(hd)
    if causal:
        logits = logits.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    ref_lse = torch.logsumexp(logits, -1)
    assert (lse_f.cpu() - ref_lse).abs().max().item() < 2e-2
    # row sums of bf16 P against two different reference maxima: |d log l| <= 2^-7
    assert (lse_f - lse_o).abs().max().item() < 2 ** -7


def test_attention_score_bound_outside_fixed_range(cuda):
    """A bound whose reference max would exceed 2^48 relative range (here
    |q.k| up to 300 at hd 64), or any key mask, keeps the running row max."""
    from hydra_amd.attention.backends.ccgqa.ops import (MASK_KEY_PADDING, attention_forward,
                                                        qk_norm_score_bound)

    q, k, v = _normed_qkv(1, 4, 1, 256, 64, 300.0, seed=5)
    dev = lambda t: t.to(cuda, torch.bfloat16)
    out, _ = attention_forward(dev(q), dev(k), dev(v), causal=True,
                               score_bound=qk_norm_score_bound(300.0))
    assert max_rel_err(out.cpu(), occ.attention(q, k, v, causal=True)) < 2e-2
    q, k, v = _normed_qkv(1, 4, 1, 256, 64, 2.0, seed=6)
    mask = torch.ones(1, 256, dtype=torch.long)
    mask[0, 10:90] = 0
    out, _ = attention_forward(dev(q), dev(k), dev(v), causal=True, key_mask=mask.to(cuda),
                               mask_mode=MASK_KEY_PADDING, score_bound=qk_norm_score_bound(2.0))
    ref = occ.attention_key_padding(q, k, v, causal=True, mask=mask)
    assert max_rel_err(out.cpu(), ref) < 2e-2


def _vt_rows(t):
    """The same values with the keys contiguous ([.., hd, S] storage), the
    layout CCGQA's prep kernel writes V in."""
    return t.transpose(2, 3).contiguous().transpose(2, 3)


VT_CASES = [
    # B, Hq, Hkv, S, hd; S % 8 == 0, so V^T rows are read as they are
    (4, 4, 1, 520, 64),
    (2, 8, 2, 136, 16),
    (1, 4, 4, 264, 32),
    (2, 8, 1, 104, 128),
    (1, 4, 2, 8, 64),
    (3, 6, 3, 72, 16),
    (1, 8, 1, 1000, 64),
    (2, 28, 4, 264, 16),  # config 5's heads: groups of 7, head_dim 16
]
VT_MODES = [(True, "none"), (False, "none"), (True, "key_padding"), (False, "key_padding"),
            (True, "reference")]


@pytest.mark.parametrize("sched", ["kp", "streamk"])
@pytest.mark.parametrize("mode", VT_MODES, ids=[f"{c}-{m}" for c, m in VT_MODES])
@pytest.mark.parametrize("case", VT_CASES, ids=[str(c) for c in VT_CASES])
def test_attention_vt_rows_schedules(cuda, monkeypatch, case, mode, sched):
    """V given as V^T rows: the key-split workgroups (one per item; kp) and
    the stream-K schedule both give the oracle's result and LSE, for every
    mask mode, with S not a multiple of the 64-key tile."""
    from hydra_amd.attention.backends.ccgqa.ops import (MASK_KEY_PADDING, MASK_NONE,
                                                        MASK_REFERENCE_SDPA, attention_forward)

    causal, mname = mode
    B, Hq, Hkv, S, hd = case
    monkeypatch.setenv("HYDRA_ATTN_SCHED", sched)
    q, k, v = _qkv(B, Hq, Hkv, S, hd, seed=S + hd + 1)
    mask = None
    if mname != "none":
        g = torch.Generator().manual_seed(S + 1)
        mask = (torch.rand(B, S, generator=g) > 0.25).long()
        mask[:, 0] = 1
        mask[0, 1:70] = 0
    mm = {"none": MASK_NONE, "key_padding": MASK_KEY_PADDING, "reference": MASK_REFERENCE_SDPA}[mname]
    dev = lambda t: t.to(cuda, torch.bfloat16)
    out, lse = attention_forward(dev(q), dev(k), _vt_rows(dev(v)), causal=causal,
                                 key_mask=None if mask is None else mask.to(cuda), mask_mode=mm,
                                 want_lse=True)
    out2, lse2 = attention_forward(dev(q), dev(k), _vt_rows(dev(v)), causal=causal,
                                   key_mask=None if mask is None else mask.to(cuda), mask_mode=mm,
                                   want_lse=True)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    if mname == "key_padding":
        ref = occ.attention_key_padding(q, k, v, causal=causal, mask=mask)
    else:
        ref = occ.attention(q, k, v, causal=causal, mask=mask)
    assert max_rel_err(out.cpu(), ref) < 2e-2
    if mname == "none":
        G = Hq // Hkv
        logits = (q @ k.repeat_interleave(G, 1).transpose(-1, -2)) / math.sqrt(hd)
        if causal:
            logits = logits.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
        assert (lse.cpu() - torch.logsumexp(logits, -1)).abs().max().item() < 2e-2


@pytest.mark.parametrize("pad,shift", [(68, 0), (64, 4), (72, 0)])
def test_attention_vt_rows_output_views(cuda, monkeypatch, pad, shift):
    """The key-split kernel at hd 64 stores whole 16-byte row chunks, so it
    takes an output view only with 16-byte aligned rows; other views (row
    stride 68, or a base 8 bytes past alignment) run the stream-K kernel.
    Every view gets the oracle's result, and the padding around it is not
    written."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    monkeypatch.setenv("HYDRA_ATTN_SCHED", "kp")
    B, Hq, Hkv, S, hd = 2, 4, 1, 264, 64
    q, k, v = _qkv(B, Hq, Hkv, S, hd, seed=77)
    dev = lambda t: t.to(cuda, torch.bfloat16)
    buf = torch.full((B * S * Hq * pad + shift,), 7.0, device=cuda, dtype=torch.bfloat16)
    view = buf[shift:].view(B, S, Hq, pad)[..., :hd].transpose(1, 2)
    out, _ = attention_forward(dev(q), dev(k), _vt_rows(dev(v)), causal=True, out=view)
    ref = occ.attention(q, k, v, causal=True)
    assert max_rel_err(view.float().cpu(), ref) < 2e-2
    full = buf[shift:].view(B, S, Hq, pad)
    if pad > hd:
        assert bool((full[..., hd:] == 7.0).all())
    if shift:
        assert bool((buf[:shift] == 7.0).all())


FIXED_VT_CASES = [
    # B, Hq, Hkv, S, hd, temperature, causal
    (4, 4, 1, 512, 64, 1.0, True),
    (2, 8, 2, 304, 16, 4.0, True),
    (1, 4, 4, 264, 32, 5.66, False),
    (2, 8, 1, 104, 128, 11.3, True),
    (1, 2, 1, 64, 64, -8.0, False),
    (1, 4, 1, 2048, 64, 40.0, True),
    (2, 28, 4, 304, 16, 4.0, True),  # config 5's heads, temperature sqrt(16)
]


@pytest.mark.parametrize("sched", ["kp", "streamk"])
@pytest.mark.parametrize("case", FIXED_VT_CASES, ids=[str(c) for c in FIXED_VT_CASES])
def test_attention_fixed_vt_rows(cuda, monkeypatch, case, sched):
    """Bounded scores with V^T rows, under both schedules: oracle result,
    online-max result and closed-form LSE."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward, qk_norm_score_bound

    B, Hq, Hkv, S, hd, temp, causal = case
    monkeypatch.setenv("HYDRA_ATTN_SCHED", sched)
    q, k, v = _normed_qkv(B, Hq, Hkv, S, hd, temp, seed=S + hd + 2)
    dev = lambda t: t.to(cuda, torch.bfloat16)
    out_f, lse_f = attention_forward(dev(q), dev(k), _vt_rows(dev(v)), causal=causal, want_lse=True,
                                     score_bound=qk_norm_score_bound(temp))
    out_o, lse_o = attention_forward(dev(q), dev(k), _vt_rows(dev(v)), causal=causal, want_lse=True)
    ref = occ.attention(q, k, v, causal=causal)
    assert max_rel_err(out_f.cpu(), ref) < 2e-2
    assert max_rel_err(out_o.cpu(), ref) < 2e-2
    G = Hq // Hkv
    logits = (q @ k.repeat_interleave(G, 1).transpose(-1, -2)) / math.sqrt(hd)
    if causal:
        logits = logits.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    ref_lse = torch.logsumexp(logits, -1)
    assert (lse_f.cpu() - ref_lse).abs().max().item() < 2e-2
    assert (lse_f - lse_o).abs().max().item() < 2 ** -7


@pytest.mark.parametrize("vt", [False, True])
@pytest.mark.parametrize("tdtype", [torch.bfloat16, torch.float32])
def test_attention_bound_from_device_temperature(cuda, vt, tdtype):
    """bound_temperature: the kernel takes qk_norm_score_bound of the
    temperature on the device.  Inside the fixed range it gives exactly the
    host-bound result; outside (|q.k| up to 300) exactly the running-max
    result."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward, qk_norm_score_bound

    dev = lambda t: t.to(cuda, torch.bfloat16)
    vv = (lambda t: _vt_rows(dev(t))) if vt else dev
    for temp in (2.0, 300.0):
        q, k, v = _normed_qkv(1, 4, 1, 512, 64, temp, seed=7)
        t = torch.full((1,), temp, dtype=tdtype, device=cuda)
        out_d, lse_d = attention_forward(dev(q), dev(k), vv(v), causal=True, want_lse=True,
                                         bound_temperature=t)
        out_h, lse_h = attention_forward(dev(q), dev(k), vv(v), causal=True, want_lse=True,
                                         score_bound=qk_norm_score_bound(temp))
        assert torch.equal(out_d, out_h) and torch.equal(lse_d, lse_h)
        assert max_rel_err(out_d.cpu(), occ.attention(q, k, v, causal=True)) < 2e-2


def test_attention_device_bound_follows_temperature_in_graph(cuda):
    """A HIP graph captured with bound_temperature reads the temperature at
    every replay: raising it past the fixed range afterwards switches the
    replays to the running-max path (whose result differs in the last bits)."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward

    dev = lambda t: t.to(cuda, torch.bfloat16)
    q, k, v = (dev(x) for x in _normed_qkv(1, 4, 1, 512, 64, 2.0, seed=8))
    t = torch.full((1,), 2.0, dtype=torch.float32, device=cuda)
    out = torch.empty_like(q)
    want_fixed, _ = attention_forward(q, k, v, causal=True, score_bound=2.06)
    want_online, _ = attention_forward(q, k, v, causal=True)
    assert not torch.equal(want_fixed, want_online)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        attention_forward(q, k, v, causal=True, out=out, bound_temperature=t)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        attention_forward(q, k, v, causal=True, out=out, bound_temperature=t)
    for temp, want in ((2.0, want_fixed), (1000.0, want_online), (2.0, want_fixed)):
        t.fill_(temp)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), temp
