"""Pin the CPU oracle (oracle/attention.py) before trusting it as the checker.

Checks, per oracle function:
* golden vectors regenerated from the reference tests' seeded fixtures, with
  outputs from a scalar float64 brute force (tests/golden/brute.py);
* the reference's known-answer tests re-expressed (exact 1.0 / 9.0 outputs,
  comparison with scaled_dot_product_attention, window boundaries);
* torch's scaled_dot_product_attention with independently built masks;
* closed forms and invariants;
* planted mistakes in a copy of the oracle that these checks must catch.
"""

import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from tests.golden import brute
from tests.golden.make_golden import tts_seed17_inputs
from voiceagent_amd import workloads
from voiceagent_amd.audio import batcher

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _npz(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


# --------------------------------------------------------------- golden vectors
def test_tts_seed17_inputs_match_fixture():
    g = _npz("tts_seed17.npz")
    q, kp, vp, table, lens, valid, nk, nv = tts_seed17_inputs()
    assert np.array_equal(kp.numpy(), g["k_pool"]) and np.array_equal(vp.numpy(), g["v_pool"])
    assert np.array_equal(nk.numpy(), g["new_key"]) and np.array_equal(nv.numpy(), g["new_value"])


def test_paged_decode_matches_tts_seed17_golden():
    # Reference fixture: tests/test_qwen_tts_paged_attention_kernel.py:16-57 (HND, page 2, D 4).
    g = _npz("tts_seed17.npz")
    q = torch.from_numpy(g["q"])[:, :, 0]
    out = oracle.paged_decode(q, torch.from_numpy(g["k_pool"]), torch.from_numpy(g["v_pool"]),
                              torch.from_numpy(g["page_table"]), torch.from_numpy(g["seq_lens"]),
                              0.5, layout=oracle.HND, valid_mask=torch.from_numpy(g["valid"]),
                              compute_dtype=torch.float64)
    np.testing.assert_allclose(out.numpy(), g["expected"], rtol=0, atol=1e-12)


def test_paged_decode_matches_reference_test_formulation():
    # The reference test's own expected value: -inf masking of the valid mask
    # (test_qwen_tts_paged_attention_kernel.py:43-57).
    q, kp, vp, table, lens, valid, _, _ = tts_seed17_inputs()
    expected = []
    for row in range(2):
        positions = torch.arange(int(lens[row]))
        pages = table[row, positions // 2]
        offsets = positions % 2
        keys = kp[pages, :, offsets, :].permute(1, 0, 2).unsqueeze(0).repeat_interleave(2, dim=1)
        values = vp[pages, :, offsets, :].permute(1, 0, 2).unsqueeze(0).repeat_interleave(2, dim=1)
        scores = torch.matmul(q[row:row + 1], keys.transpose(-1, -2)) / 2.0
        scores = scores.masked_fill(~valid[row, :int(lens[row])].view(1, 1, 1, -1), -torch.inf)
        expected.append(torch.softmax(scores, dim=-1) @ values)
    expected = torch.cat(expected, dim=0)[:, :, 0]
    out = oracle.paged_decode(q[:, :, 0], kp, vp, table, lens, 0.5, layout=oracle.HND,
                              valid_mask=valid)
    assert torch.allclose(out, expected, atol=1e-6)


def test_write_current_kv_matches_fused_golden():
    # test_qwen_tts_paged_attention_kernel.py:144-177: the new row lands at seq_len - 1.
    g = _npz("tts_seed17.npz")
    kp, vp = oracle.write_current_kv(torch.from_numpy(g["k_pool"]), torch.from_numpy(g["v_pool"]),
                                     torch.from_numpy(g["page_table"]),
                                     torch.from_numpy(g["seq_lens"]),
                                     torch.from_numpy(g["new_key"])[:, :, 0],
                                     torch.from_numpy(g["new_value"])[:, :, 0])
    assert np.array_equal(kp.numpy(), g["k_pool_fused"])
    assert np.array_equal(vp.numpy(), g["v_pool_fused"])
    out = oracle.paged_decode(torch.from_numpy(g["q"])[:, :, 0], kp, vp,
                              torch.from_numpy(g["page_table"]), torch.from_numpy(g["seq_lens"]),
                              0.5, layout=oracle.HND, valid_mask=torch.from_numpy(g["valid"]),
                              compute_dtype=torch.float64)
    np.testing.assert_allclose(out.numpy(), g["expected_fused"], rtol=0, atol=1e-12)


def test_paged_decode_matches_cfg1_golden():
    g = _npz("cfg1_decode.npz")
    lens = workloads.cfg1_lens(0)
    assert lens == g["lens"].tolist()
    b = workloads.make_decode_batch(lens, num_blocks=128, dtype=torch.float32, seed=0)
    assert np.array_equal(b.block_tables.numpy(), g["block_tables"])
    assert math.isclose(float(b.q.double().sum()), float(g["q_sum"]), rel_tol=0, abs_tol=1e-9)
    assert math.isclose(float(b.k_pools[0].double().sum()), float(g["k_sum"]), abs_tol=1e-6)
    out32 = oracle.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables,
                                b.context_lens, b.scale)
    out64 = oracle.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables,
                                b.context_lens, b.scale, compute_dtype=torch.float64)
    np.testing.assert_allclose(out64.numpy(), g["expected"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(out32.numpy(), g["expected"], rtol=0, atol=1e-5)


# ---------------------------------------------------------------- known answers
def test_integer_known_answers():
    # test_qwen_tts_outer_varlen_attention.py:54-66: constant K/V gives exactly 1.0 and 9.0.
    kp = torch.zeros(8, 1, 2, 1)
    vp = torch.zeros(8, 1, 2, 1)
    table = torch.tensor([[0, 1], [2, 3]])
    kp[0:2] = 1.0
    vp[0:2] = 1.0
    kp[2:4] = 9.0
    vp[2:4] = 9.0
    out = oracle.paged_decode(torch.ones(2, 1, 1), kp, vp, table, torch.tensor([4, 4]), 1.0,
                              layout=oracle.HND)
    assert out[0].item() == 1.0 and out[1].item() == 9.0


def test_matches_sdpa_known_answer():
    # test_qwen_tts_outer_varlen_attention.py:24-48: keys [1,2,3] (values x10), query 2;
    # keys [100, 200], query 150; against scaled_dot_product_attention.
    kp = torch.zeros(8, 1, 2, 1)
    vp = torch.zeros(8, 1, 2, 1)
    table = torch.tensor([[0, 1], [2, 3]])
    for t, val in enumerate([1.0, 2.0, 3.0]):
        kp[t // 2, 0, t % 2, 0] = val
        vp[t // 2, 0, t % 2, 0] = 10 * val
    for t, val in enumerate([100.0, 200.0]):
        kp[2 + t // 2, 0, t % 2, 0] = val
        vp[2 + t // 2, 0, t % 2, 0] = 10 * val
    q = torch.tensor([[[2.0]], [[150.0]]])
    out = oracle.paged_decode(q, kp, vp, table, torch.tensor([3, 2]), 1.0, layout=oracle.HND)
    ka = torch.tensor([1.0, 2.0, 3.0]).view(1, 1, 3, 1)
    kb = torch.tensor([100.0, 200.0]).view(1, 1, 2, 1)
    ea = torch.nn.functional.scaled_dot_product_attention(q[0].view(1, 1, 1, 1), ka, ka * 10)
    eb = torch.nn.functional.scaled_dot_product_attention(q[1].view(1, 1, 1, 1), kb, kb * 10)
    assert torch.allclose(out[0], ea.view(1, 1), atol=1e-5)
    assert torch.allclose(out[1], eb.view(1, 1), atol=1e-3)


def test_window_boundaries_known_answers():
    # tests/test_units.py:33-45 and :74-110 of the reference.
    def official(n):
        leave = n % 100
        feat = (leave - 1) // 2 + 1
        return ((feat - 1) // 2 + 1 - 1) // 2 + 1 + (n // 100) * 13

    assert all(batcher.num_audio_tokens(f) == official(f) for f in range(1, 6000))
    assert batcher.attention_window_tokens(800) == 104
    assert batcher.build_window_boundaries([46, 26, 95], 104) == [0, 46, 72, 167]
    assert batcher.build_window_boundaries([250], 104) == [0, 104, 208, 250]
    assert batcher.build_window_boundaries([208], 104) == [0, 104, 208]
    cu, widest = batcher.window_cu_seqlens([46, 26, 95], 104)
    assert cu.dtype == torch.int32 and cu.tolist() == [0, 46, 72, 167] and widest == 95


# -------------------------------------------------------------- closed forms
def _rand_pool(gen, nb=12, bs=4, hkv=2, d=8):
    return (torch.randn(nb, bs, hkv, d, generator=gen, dtype=torch.float64),
            torch.randn(nb, bs, hkv, d, generator=gen, dtype=torch.float64))


def test_decode_closed_forms():
    gen = torch.Generator().manual_seed(5)
    kp, vp = _rand_pool(gen)
    table = torch.tensor([[7, 2, 9], [4, 0, 11]])
    q = torch.randn(2, 4, 8, generator=gen, dtype=torch.float64)
    # single key -> that key's value row
    out = oracle.paged_decode(q, kp, vp, table, torch.tensor([1, 1]), 0.3,
                              compute_dtype=torch.float64)
    assert torch.allclose(out[0], vp[7, 0].repeat_interleave(2, dim=0))
    assert torch.allclose(out[1], vp[4, 0].repeat_interleave(2, dim=0))
    # zero query -> mean of the values
    out = oracle.paged_decode(torch.zeros_like(q), kp, vp, table, torch.tensor([10, 7]), 0.3,
                              compute_dtype=torch.float64)
    rows = oracle.gather_rows(vp, table[0], torch.arange(10))
    assert torch.allclose(out[0], rows.mean(0).repeat_interleave(2, dim=0))
    # constant values -> that constant
    vc = torch.full_like(vp, 2.5)
    out = oracle.paged_decode(q, kp, vc, table, torch.tensor([10, 7]), 0.3,
                              compute_dtype=torch.float64)
    assert torch.allclose(out, torch.full_like(out, 2.5))


def test_decode_block_table_permutation_invariance():
    gen = torch.Generator().manual_seed(6)
    kp, vp = _rand_pool(gen)
    table = torch.tensor([[7, 2, 9], [4, 0, 11]])
    q = torch.randn(2, 4, 8, generator=gen, dtype=torch.float64)
    lens = torch.tensor([11, 9])
    base = oracle.paged_decode(q, kp, vp, table, lens, 0.3, compute_dtype=torch.float64)
    perm = torch.randperm(kp.shape[0], generator=gen)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    out = oracle.paged_decode(q, kp[perm], vp[perm], inv[table], lens, 0.3,
                              compute_dtype=torch.float64)
    assert torch.allclose(out, base)


def test_decode_gqa_against_brute_force():
    gen = torch.Generator().manual_seed(8)
    kp, vp = _rand_pool(gen, hkv=2)
    table = torch.tensor([[7, 2, 9], [4, 0, 11]])
    q = torch.randn(2, 6, 8, generator=gen, dtype=torch.float64)  # G = 3
    lens = [9, 12]
    valid = torch.tensor([[True] * 3 + [False] * 2 + [True] * 4, [False, True] * 4 + [True]])
    out = oracle.paged_decode(q, kp, vp, table, torch.tensor(lens), 0.7, valid_mask=valid,
                              compute_dtype=torch.float64)
    ref = brute.paged_decode(q.tolist(), kp.tolist(), vp.tolist(), table.tolist(), lens, 0.7,
                             valid=valid.tolist())
    assert np.allclose(out.numpy(), np.array(ref), atol=1e-12)


def test_decode_fully_masked_row_is_zero():
    gen = torch.Generator().manual_seed(9)
    kp, vp = _rand_pool(gen)
    table = torch.tensor([[1, 2, 3]])
    valid = torch.zeros(1, 12, dtype=torch.bool)
    out = oracle.paged_decode(torch.randn(1, 4, 8, dtype=torch.float64), kp, vp, table,
                              torch.tensor([6]), 1.0, valid_mask=valid,
                              compute_dtype=torch.float64)
    assert torch.count_nonzero(out) == 0


def test_decode_tts_bounds_closed_forms():
    # key_limit (the Triton kernel's MAX_SEQ_LEN = kernel_seq_len) and
    # table_read_width (num_page_slots = kernel_page_count) against closed
    # forms: with all keys zero the softmax is uniform, so the output is the
    # mean of the attended value rows.
    bs, hkv, d = 4, 2, 8
    kp = torch.zeros(16, bs, hkv, d, dtype=torch.float64)
    vp = torch.zeros(16, bs, hkv, d, dtype=torch.float64)
    for blk in range(16):
        for off in range(bs):
            vp[blk, off] = 100.0 * blk + off  # row value names its slot
    table = torch.tensor([[5, 9, 3, 12, 7]])
    q = torch.randn(1, 4, d, dtype=torch.float64)
    vals = lambda blocks: [100.0 * blk + off for blk in blocks for off in range(bs)]  # noqa: E731
    real = vals([5, 9, 3, 12, 7])
    # key_limit 9 of a 17-token row: the mean of the first nine slots
    out = oracle.paged_decode(q, kp, vp, table, torch.tensor([17]), 0.5, key_limit=9,
                              compute_dtype=torch.float64)
    assert torch.allclose(out, torch.full_like(out, sum(real[:9]) / 9))
    # table_read_width 2: tokens of columns 2.. read block 0 (values 0..3)
    out = oracle.paged_decode(q, kp, vp, table, torch.tensor([18]), 0.5, table_read_width=2,
                              compute_dtype=torch.float64)
    expect = (sum(real[:8]) + sum(vals([0, 0, 0])[:10])) / 18
    assert torch.allclose(out, torch.full_like(out, expect))


def test_decode_masked_nonfinite_values_are_dropped():
    # A masked token whose K and V rows are non-finite counts as absent:
    # the same as attending the unmasked tokens only (gathered apart here).
    gen = torch.Generator().manual_seed(12)
    kp, vp = _rand_pool(gen)
    table = torch.tensor([[3, 8, 1]])
    q = torch.randn(1, 4, 8, generator=gen, dtype=torch.float64)
    valid = torch.tensor([[True, False, True, True, False, True, True, True, True, False, True]])
    kbad, vbad = kp.clone(), vp.clone()
    for t in (1, 4, 9):
        kbad[table[0, t // 4], t % 4] = float("nan")
        vbad[table[0, t // 4], t % 4] = float("inf")
    out = oracle.paged_decode(q, kbad, vbad, table, torch.tensor([11]), 0.4, valid_mask=valid,
                              compute_dtype=torch.float64)
    keep = [t for t in range(11) if valid[0, t]]
    keys = oracle.gather_rows(kp, table[0], torch.tensor(keep))  # [n, Hkv, D]
    values = oracle.gather_rows(vp, table[0], torch.tensor(keep))
    ref = torch.nn.functional.scaled_dot_product_attention(
        q[0].unsqueeze(1), keys.permute(1, 0, 2).repeat_interleave(2, 0),
        values.permute(1, 0, 2).repeat_interleave(2, 0), scale=0.4)
    assert torch.isfinite(out).all()
    assert torch.allclose(out[0], ref[:, 0])


def test_store_kvcache_closed_form():
    gen = torch.Generator().manual_seed(10)
    kc = torch.randn(6, 4, 2, 8, generator=gen)
    vc = torch.randn(6, 4, 2, 8, generator=gen)
    key = torch.randn(5, 2, 8, generator=gen)
    val = torch.randn(5, 2, 8, generator=gen)
    slots = torch.tensor([3, -1, 22, 0, 9])
    k2, v2 = oracle.store_kvcache(key, val, kc, vc, slots)
    flat_k, flat_v = kc.clone().view(-1, 16), vc.clone().view(-1, 16)
    for i, s in enumerate(slots.tolist()):
        if s != -1:
            flat_k[s] = key[i].reshape(-1)
            flat_v[s] = val[i].reshape(-1)
    assert torch.equal(k2.view(-1, 16), flat_k) and torch.equal(v2.view(-1, 16), flat_v)
    untouched = torch.ones(24, dtype=torch.bool)
    untouched[[3, 22, 0, 9]] = False
    assert torch.equal(k2.view(-1, 16)[untouched], kc.view(-1, 16)[untouched])


# ---------------------------------------------------------------------- varlen
def _sdpa_reference(q, k, v, keep, scale):
    """float64 SDPA per sequence with an explicit boolean mask [Hq, ql, kl]."""
    return torch.nn.functional.scaled_dot_product_attention(
        q.permute(1, 0, 2).unsqueeze(0), k.permute(1, 0, 2).unsqueeze(0),
        v.permute(1, 0, 2).unsqueeze(0), attn_mask=keep.unsqueeze(0), scale=scale,
    )[0].permute(1, 0, 2)


def test_causal_varlen_against_sdpa():
    gen = torch.Generator().manual_seed(11)
    lens = [1, 5, 17]
    total = sum(lens)
    q = torch.randn(total, 4, 8, generator=gen, dtype=torch.float64)
    k = torch.randn(total, 2, 8, generator=gen, dtype=torch.float64)
    v = torch.randn(total, 2, 8, generator=gen, dtype=torch.float64)
    cu = torch.tensor([0, 1, 6, 23], dtype=torch.int32)
    out = oracle.varlen_attention(q, k, v, cu, cu, 0.4, True, compute_dtype=torch.float64)
    for s in range(3):
        a, b = int(cu[s]), int(cu[s + 1])
        n = b - a
        keep = torch.tril(torch.ones(n, n, dtype=torch.bool)).expand(4, n, n)
        ref = _sdpa_reference(q[a:b], k[a:b].repeat_interleave(2, 1), v[a:b].repeat_interleave(2, 1),
                              keep, 0.4)
        assert torch.allclose(out[a:b], ref, atol=1e-12)
    ref = brute.varlen(q.tolist(), k.tolist(), v.tolist(), cu.tolist(), cu.tolist(), 0.4, True)
    assert np.allclose(out.numpy(), np.array(ref), atol=1e-12)


def test_causal_bottom_right_with_paged_prefix():
    # q_len < k_len (prefix-cache hit): query i sees keys j <= k_len - q_len + i.
    gen = torch.Generator().manual_seed(12)
    bs, hkv, d, hq = 4, 2, 8, 4
    kp = torch.randn(10, bs, hkv, d, generator=gen, dtype=torch.float64)
    vp = torch.randn(10, bs, hkv, d, generator=gen, dtype=torch.float64)
    table = torch.tensor([[6, 1, 8, 3]])
    k_len, q_len = 14, 5
    q = torch.randn(q_len, hq, d, generator=gen, dtype=torch.float64)
    knew = torch.randn(q_len, hkv, d, generator=gen, dtype=torch.float64)
    vnew = torch.randn(q_len, hkv, d, generator=gen, dtype=torch.float64)
    cu_q = torch.tensor([0, q_len], dtype=torch.int32)
    cu_k = torch.tensor([0, k_len], dtype=torch.int32)
    out = oracle.varlen_attention(q, knew, vnew, cu_q, cu_k, 0.35, True, k_cache=kp, v_cache=vp,
                                  block_tables=table, compute_dtype=torch.float64)
    prefix = oracle.gather_rows(kp, table[0], torch.arange(k_len - q_len))
    vprefix = oracle.gather_rows(vp, table[0], torch.arange(k_len - q_len))
    keys = torch.cat([prefix, knew]).repeat_interleave(2, 1)
    values = torch.cat([vprefix, vnew]).repeat_interleave(2, 1)
    i = torch.arange(q_len).view(-1, 1)
    j = torch.arange(k_len).view(1, -1)
    keep = (j - (k_len - q_len) <= i).expand(hq, q_len, k_len)
    ref = _sdpa_reference(q, keys, values, keep, 0.35)
    assert torch.allclose(out, ref, atol=1e-12)
    # all keys from the pool (k=None) once the new rows have been stored there
    slots = [int(table[0, p // bs]) * bs + p % bs for p in range(k_len - q_len, k_len)]
    kp2, vp2 = oracle.store_kvcache(knew, vnew, kp, vp, torch.tensor(slots))
    out2 = oracle.varlen_attention(q, None, None, cu_q, cu_k, 0.35, True, k_cache=kp2,
                                   v_cache=vp2, block_tables=table, compute_dtype=torch.float64)
    assert torch.allclose(out2, ref, atol=1e-12)


def test_block_diagonal_matches_prepare_attention_mask():
    # Mask built as reference/modeling_qwen3_asr.py:649-667 (finfo.min outside the
    # windows, 0 inside), then eager softmax(QK^T * s + mask) V (:90-113).
    gen = torch.Generator().manual_seed(13)
    cu = torch.tensor(batcher.build_window_boundaries([46, 26, 95], 10), dtype=torch.int32)
    total = int(cu[-1])
    q = torch.randn(total, 3, 8, generator=gen, dtype=torch.float64)
    k = torch.randn(total, 3, 8, generator=gen, dtype=torch.float64)
    v = torch.randn(total, 3, 8, generator=gen, dtype=torch.float64)
    mask = torch.full((total, total), torch.finfo(torch.float64).min, dtype=torch.float64)
    for a, b in zip(cu[:-1].tolist(), cu[1:].tolist()):
        mask[a:b, a:b] = 0
    scores = torch.einsum("thd,shd->hts", q, k) * 0.125 + mask
    ref = torch.einsum("hts,shd->thd", torch.softmax(scores, dim=-1), v)
    out = oracle.varlen_attention(q, k, v, cu, cu, 0.125, False, compute_dtype=torch.float64)
    assert torch.allclose(out, ref, atol=1e-12)


# ------------------------------------------------------------ planted mistakes
def test_planted_mistakes_are_caught(monkeypatch):
    """Each plausible oracle bug, planted in a patched copy, must fail a pinning check."""
    g = _npz("cfg1_decode.npz")
    lens = workloads.cfg1_lens(0)
    b = workloads.make_decode_batch(lens, num_blocks=128, dtype=torch.float32, seed=0)

    def run():
        out = oracle.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables,
                                  b.context_lens, b.scale, compute_dtype=torch.float64)
        return np.abs(out.numpy() - g["expected"]).max()

    assert run() < 1e-12
    real_gather = oracle.gather_rows

    def wrong_slot(pool, table_row, positions, layout="nhd"):  # pos // bs and pos % bs swapped
        bs = pool.shape[1]
        return real_gather(pool, table_row, (positions % bs) * bs + positions // bs, layout)

    monkeypatch.setattr(oracle, "gather_rows", wrong_slot)
    assert run() > 1e-3
    monkeypatch.setattr(oracle, "gather_rows", real_gather)

    def wrong_gqa(t, repeats, dim):  # kv head h % Hkv instead of h // G
        return t.repeat(repeats, 1, 1) if dim == 0 else t

    orig = torch.Tensor.repeat_interleave
    monkeypatch.setattr(torch.Tensor, "repeat_interleave",
                        lambda self, r, dim=None: wrong_gqa(self, r, dim))
    assert run() > 1e-3
    monkeypatch.setattr(torch.Tensor, "repeat_interleave", orig)
    assert run() < 1e-12


# ------------------------------------------------------------ q/k prologue
def _rope_complex(x, positions, base):
    """Independent float64 restatement: pair (x_i, x_{i+D/2}) as the complex
    number x_i + j x_{i+D/2}, multiplied by exp(j p base^(-2i/D))."""
    d = x.shape[-1]
    i = torch.arange(d // 2, dtype=torch.float64)
    theta = positions.double()[:, None] * base ** (-2.0 * i / d)[None, :]
    z = torch.complex(x[..., : d // 2].double(), x[..., d // 2:].double())
    r = z * torch.polar(torch.ones_like(theta), theta)[:, None, :]
    return torch.cat((r.real, r.imag), dim=-1)


def test_rms_norm_closed_forms():
    eps = 1e-6
    for c in (0.5, -3.0, 40.0):
        x = torch.full((2, 3, 128), c)
        y = oracle.rms_norm(x, torch.ones(128), eps)
        want = (1.0 if c > 0 else -1.0) / (1.0 + eps / c ** 2) ** 0.5
        assert torch.allclose(y, torch.full_like(y, want), atol=1e-6)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 4, 64, generator=g, dtype=torch.float64)
    w = torch.rand(64, generator=g, dtype=torch.float64) + 0.5
    ref = x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * w
    assert torch.allclose(oracle.rms_norm(x.float(), w.float(), eps).double(), ref, atol=1e-5)
    # bf16 input: the normalised value is rounded before the weight, as the reference does
    xb = x.to(torch.bfloat16)
    wb = w.to(torch.bfloat16)
    y = oracle.rms_norm(xb, wb, eps)
    n = (xb.float() * torch.rsqrt(xb.float().pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
    assert y.dtype == torch.bfloat16 and torch.equal(y, n * wb)
    # an fp32 weight on bf16 activations keeps the activation dtype (in-place product)
    assert oracle.rms_norm(xb, w.float(), eps).dtype == torch.bfloat16


def test_rope_matches_complex_rotation_and_identity_at_zero():
    base, d = 1_000_000.0, 128
    cs = oracle.rope_cache(d, 4096, base)
    assert cs.shape == (4096, d) and cs.dtype == torch.float32
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 3, d, generator=g)
    pos = torch.randint(0, 4096, (64,), generator=g)
    got = oracle.apply_rope(x, cs, pos).double()
    want = _rope_complex(x, pos, base)
    # fp32 angles of up to ~4096 rad: absolute error of a few 1e-4 at most
    assert (got - want).abs().max() < 2e-3
    zero = torch.zeros(64, dtype=torch.long)
    assert torch.equal(oracle.apply_rope(x, cs, zero), x)
    # rotation preserves the norm of every (i, i + D/2) pair
    pn = lambda t: t[..., : d // 2] ** 2 + t[..., d // 2:] ** 2  # noqa: E731
    assert torch.allclose(pn(got), pn(x.double()), rtol=1e-5, atol=1e-5)


def test_prologue_planted_mistakes_fail():
    base, d = 10000.0, 64
    cs = oracle.rope_cache(d, 512, base)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(32, 2, d, generator=g)
    pos = torch.randint(1, 512, (32,), generator=g)
    want = _rope_complex(x, pos, base)
    cos, sin = cs[pos].unsqueeze(1).chunk(2, dim=-1)
    a, b = x.chunk(2, dim=-1)
    flipped = torch.cat((a * cos + b * sin, b * cos - a * sin), -1)   # wrong sign
    swapped = torch.cat((b * cos - a * sin, a * cos + b * sin), -1)   # halves swapped
    for bad in (flipped, swapped):
        assert (bad.double() - want).abs().max() > 0.1
    w = torch.rand(d, generator=g) + 0.5
    assert (oracle.rms_norm(x, w, 1e-6) - oracle.rms_norm(x, torch.ones(d), 1e-6)).abs().max() > 0.1
    qn, kn = oracle.qk_norm_rope(x, x[:, :1], pos, w, w, 1e-6, cs)
    assert torch.allclose(qn.double(), _rope_complex(oracle.rms_norm(x, w, 1e-6), pos, base),
                          atol=2e-3)


# ------------------------------------------------------------------ FP8 pools
def test_fp8_quantize_known_values_of_the_ocp_e4m3_format():
    # Codes from the OCP 8-bit floating point specification (E4M3, bias 7, no
    # infinities, 0x7f/0xff NaN): exponent/mantissa fields read off by hand.
    cases = [(1.0, 0x38), (-1.0, 0xB8), (448.0, 0x7E), (-448.0, 0xFE), (2.0 ** -9, 0x01),
             (2.0 ** -6, 0x08), (7 * 2.0 ** -9, 0x07), (240.0, 0x77), (0.5, 0x30),
             (1.125, 0x39), (1.25, 0x3A), (3.5, 0x46), (0.0, 0x00)]
    x = torch.tensor([c[0] for c in cases])
    got = oracle.quantize_fp8(x, 1.0).view(torch.uint8).tolist()
    assert got == [c[1] for c in cases]
    # saturation, not NaN, past the largest finite value
    big = oracle.quantize_fp8(torch.tensor([500.0, 1e30, float("inf"), -float("inf")]), 1.0)
    assert big.view(torch.uint8).tolist() == [0x7E, 0x7E, 0x7E, 0xFE]
    # halfway cases round to the even mantissa
    ties = torch.tensor([1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 464.0 - 1e-3])
    assert oracle.quantize_fp8(ties, 1.0).view(torch.uint8).tolist() == [0x38, 0x3A, 0x00, 0x02,
                                                                         0x7E]


def test_fp8_every_finite_code_round_trips_and_scales():
    codes = torch.arange(256, dtype=torch.uint8)
    finite = codes[(codes & 0x7F) != 0x7F]  # 0x7f / 0xff are NaN
    vals = oracle.dequantize_fp8(finite.view(oracle.FP8), 1.0)
    assert torch.isfinite(vals).all()
    assert torch.equal(oracle.quantize_fp8(vals, 1.0).view(torch.uint8), finite)
    # the positive codes are ordered like their values
    pos = torch.arange(0x00, 0x7F, dtype=torch.uint8)
    pv = oracle.dequantize_fp8(pos.view(oracle.FP8), 1.0)
    assert torch.all(pv[1:] > pv[:-1])
    # a power-of-two scale moves values without changing codes
    assert torch.equal(oracle.quantize_fp8(vals * 0.25, 0.25).view(torch.uint8), finite)
    # quantisation error is at most half a step: 2^-4 relative in the normal range
    x = torch.randn(4096, generator=torch.Generator().manual_seed(2)) * 30
    r = oracle.dequantize_fp8(oracle.quantize_fp8(x, 0.7), 0.7)
    normal = x.abs() > 2.0 ** -6 * 0.7
    assert ((r - x).abs()[normal] <= x.abs()[normal] * 2.0 ** -4 + 1e-7).all()


def test_fp8_decode_on_grid_values_equals_the_16_bit_decode():
    # K/V drawn from the e4m3 grid are stored exactly by FP8 and by bf16:
    # the FP8 decode (scale 1) must equal the decode of the bf16 pools, which
    # the golden vectors above pin.
    gen = torch.Generator().manual_seed(21)
    codes = torch.randint(0, 0x7F, (12, 4, 2, 8), generator=gen, dtype=torch.uint8)
    sign = torch.randint(0, 2, codes.shape, generator=gen, dtype=torch.uint8) << 7
    kc = (codes | sign).view(oracle.FP8)
    vc = torch.randint(0, 0x7F, (12, 4, 2, 8), generator=gen, dtype=torch.uint8).view(oracle.FP8)
    kb = oracle.dequantize_fp8(kc, 1.0).to(torch.bfloat16)
    vb = oracle.dequantize_fp8(vc, 1.0).to(torch.bfloat16)
    assert torch.equal(kb.float(), oracle.dequantize_fp8(kc, 1.0))  # bf16 holds them exactly
    table = torch.tensor([[3, 7, 1], [5, 0, 11]])
    lens = torch.tensor([10, 7])
    q = torch.randn(2, 4, 8, generator=gen) * 0.05
    a = oracle.paged_decode(q, kc, vc, table, lens, 0.3)
    b = oracle.paged_decode(q, kb, vb, table, lens, 0.3)
    assert torch.equal(a, b)
    # scales: K scale multiplies the logits, V scale the output
    a2 = oracle.paged_decode(q, kc, vc, table, lens, 0.3, k_scale=2.0, v_scale=0.5)
    b2 = oracle.paged_decode(q * 2.0, kb, vb, table, lens, 0.3) * 0.5
    assert torch.allclose(a2, b2, atol=1e-6)
    # a store into an FP8 pool writes the quantised rows and nothing else
    key = torch.randn(3, 2, 8, generator=gen)
    ek, ev = oracle.store_kvcache(key, key * 2, kc, vc, torch.tensor([5, -1, 17]), k_scale=0.5,
                                  v_scale=4.0)
    assert torch.equal(ek[1, 1].view(torch.uint8), oracle.quantize_fp8(key[0], 0.5).view(torch.uint8))
    assert torch.equal(ev[4, 1].view(torch.uint8),
                       oracle.quantize_fp8(key[2] * 2, 4.0).view(torch.uint8))
    untouched = torch.ones(12, 4, dtype=torch.bool)
    untouched[1, 1] = untouched[4, 1] = False
    assert torch.equal(ek.view(torch.uint8)[untouched], kc.view(torch.uint8)[untouched])
