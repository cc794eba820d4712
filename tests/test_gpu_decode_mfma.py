"""The matrix-core decode path (16-bit K/V, block size a multiple of 16, no key
mask) against the CPU oracle: block sizes, tile edges, context partitions,
zero-length rows, unmapped blocks, the TTS page layout with the fused current-row
write, and contexts long enough to refill a wave's block-id prefetch.

Tolerance: max-abs 2e-2 for bf16/fp16 against the oracle in fp32; pools written
by the fused store are compared bit for bit.
"""

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops
from voiceagent_amd.agent import paged_attention_decode

pytestmark = pytest.mark.gpu

TOL = 2e-2
EDGE_LENS = [1, 15, 16, 17, 31, 63, 64, 65, 130, 255, 256, 257, 700]


def _err(out, ref):
    return (out.float().cpu() - ref.float()).abs().max().item()


def _nhd_case(lens, bs, dtype, hq=16, hkv=8, d=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    need = [(n + bs - 1) // bs for n in lens]
    nb = sum(need) + 4
    perm = torch.randperm(nb, generator=g).tolist()
    width = max(need)
    rows, cur = [], 0
    for m in need:
        rows.append(perm[cur:cur + m] + [-1] * (width - m))
        cur += m
    table = torch.tensor(rows, dtype=torch.int32)
    kp = (torch.randn(nb, bs, hkv, d, generator=g) * 0.5).to(dtype)
    vp = (torch.randn(nb, bs, hkv, d, generator=g) * 0.5).to(dtype)
    q = torch.randn(len(lens), hq, d, generator=g).to(dtype)
    return q, kp, vp, table, torch.tensor(lens, dtype=torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bs", [16, 32, 48, 64])
def test_block_sizes_and_tile_edges(dev, dtype, bs):
    q, kp, vp, table, lt = _nhd_case(EDGE_LENS, bs, dtype, seed=bs)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=max(EDGE_LENS), scale=128 ** -0.5)
    ref = oracle.paged_decode(q, kp, vp, table, lt, 128 ** -0.5)
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("split", [64, 256, 512, 2048])
def test_partitions_and_merge(dev, split):
    lens = [1, 16, 300, 1500, 4000]
    q, kp, vp, table, lt = _nhd_case(lens, 16, torch.bfloat16, seed=split)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=max(lens), scale=128 ** -0.5, split_tokens=split)
    ref = oracle.paged_decode(q, kp, vp, table, lt, 128 ** -0.5)
    assert _err(out, ref) <= TOL


def test_zero_length_rows_and_unmapped_blocks(dev):
    q, kp, vp, table, _ = _nhd_case([40, 40, 40], 16, torch.bfloat16, seed=3)
    table[1, 1] = 999999  # unmapped: its 16 tokens are masked, never read
    table[2, 2] = -1
    lt = torch.tensor([0, 40, 40], dtype=torch.int32)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=40, scale=0.1).cpu()
    assert torch.count_nonzero(out[0]) == 0
    keep = torch.ones(3, 40, dtype=torch.bool)
    keep[1, 16:32] = False
    keep[2, 32:40] = False
    safe = table.clone()
    safe[1, 1] = 0
    safe[2, 2] = 0
    ref = oracle.paged_decode(q, kp, vp, safe, lt, 0.1, valid_mask=keep)
    assert _err(out[1:], ref[1:]) <= TOL


def test_prefetch_refill_past_64_tiles_per_wave(dev):
    # One partition of 20000 tokens: each of the 8 waves owns ~156 tiles, so the
    # block-id prefetch (64 tiles per refill) is refilled twice.
    lens = [20000, 37]
    q, kp, vp, table, lt = _nhd_case(lens, 16, torch.bfloat16, seed=21)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=20000, scale=128 ** -0.5, split_tokens=20480)
    ref = oracle.paged_decode(q, kp, vp, table, lt, 128 ** -0.5)
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("page", [16, 32])
def test_tts_page_layout_with_fused_write(dev, page):
    # TTS pool [pages, Hkv, page_size, D], int64 tables, no key mask: the
    # current row is written at seq_len - 1 and attended in the same launch.
    g = torch.Generator().manual_seed(page)
    lens = torch.tensor([1, page, page + 1, 3 * page - 2], dtype=torch.long)
    pages_needed = [(int(n) + page - 1) // page for n in lens]
    P = sum(pages_needed) + 3
    perm = torch.randperm(P, generator=g).tolist()
    width = max(pages_needed)
    rows, cur = [], 0
    for m in pages_needed:
        rows.append(perm[cur:cur + m] + [-1] * (width - m))
        cur += m
    table = torch.tensor(rows, dtype=torch.long)
    kp = torch.randn(P, 8, page, 128, generator=g).to(torch.bfloat16)
    vp = torch.randn(P, 8, page, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(4, 16, 1, 128, generator=g).to(torch.bfloat16)
    nk = torch.randn(4, 8, 1, 128, generator=g).to(torch.bfloat16)
    nv = torch.randn(4, 8, 1, 128, generator=g).to(torch.bfloat16)
    ek, ev = oracle.write_current_kv(kp, vp, table, lens, nk[:, :, 0], nv[:, :, 0])
    kd, vd = kp.to(dev), vp.to(dev)
    out = paged_attention_decode(q.to(dev), kd, vd, table.to(dev), lens.to(dev),
                                 new_key=nk.to(dev), new_value=nv.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.paged_decode(q[:, :, 0], ek, ev, table, lens, 128 ** -0.5, layout=oracle.HND)
    assert _err(out[:, :, 0], ref) <= TOL


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("lens", [[5, 900], [1, 2, 17, 1000]])
def test_fixed_partitions_from_a_short_bound(dev, masked, lens):
    # An automatic split under a short max_seq_len (here 1024) uses fixed
    # partitions whose first tiles go out before the lengths arrive: short
    # contexts leave partitions wholly past their end (fetched, then
    # dropped), and the current row is written and attended in the same
    # launch.
    q, kp, vp, table, lt = _nhd_case(lens, 16, torch.bfloat16, seed=len(lens) + masked)
    B = len(lens)
    g = torch.Generator().manual_seed(11)
    nk = torch.randn(B, 8, 128, generator=g).to(torch.bfloat16)
    nv = torch.randn(B, 8, 128, generator=g).to(torch.bfloat16)
    valid = (torch.rand(B, 1024, generator=g) < 0.8) if masked else None
    ek, ev = oracle.write_current_kv(kp, vp, table, lt, nk, nv, layout=oracle.NHD)
    kd, vd = kp.to(dev), vp.to(dev)
    print(f"fixed partitions lens={lens} masked={masked}", flush=True)
    out = ops.paged_decode(q.to(dev), kd, vd, table.to(dev), lt.to(dev), max_seq_len=1024,
                           scale=128 ** -0.5, new_k=nk.to(dev), new_v=nv.to(dev),
                           valid_mask=None if valid is None else valid.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.paged_decode(q, ek, ev, table, lt, 128 ** -0.5, valid_mask=valid)
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("lens,max_seq_len", [
    ([7, 300, 9000], 9000), ([9000], 9000), ([7, 300, 9000], 5000), ([20, 30], 30)])
def test_exact_bound_split(dev, dtype, lens, max_seq_len):
    # split_tokens = SPLIT_EXACT (an eager step's exact longest context) fixes
    # the partitions from max_seq_len at any length; a context longer than
    # the bound (5000 here) is still attended whole, by the last partition.
    q, kp, vp, table, lt = _nhd_case(lens, 16, dtype, seed=max_seq_len % 89 + len(lens))
    print(f"exact split lens={lens} max_seq_len={max_seq_len} {dtype}", flush=True)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=max_seq_len, scale=128 ** -0.5,
                           split_tokens=ops.SPLIT_EXACT)
    ref = oracle.paged_decode(q, kp, vp, table, lt, 128 ** -0.5)
    assert _err(out, ref) <= (TOL if dtype != torch.float32 else 1e-5)


def test_split_tokens_below_exact_is_rejected(dev):
    q, kp, vp, table, lt = _nhd_case([40, 40], 16, torch.bfloat16, seed=1)
    with pytest.raises(Exception, match="split_tokens"):
        ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                         max_seq_len=40, scale=0.1, split_tokens=-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("max_seq_len", [4000, 65536, 100])
def test_max_seq_len_as_upper_bound(dev, dtype, max_seq_len):
    # A decode graph is captured with max_seqlen_k = max_model_len
    # (qwen_asr_vllm/engine/graph_runner.py:85-93): the automatic split sizes
    # each context's partitions from its own length, so an upper bound (or an
    # underestimate) gives the same result as the exact maximum.
    lens = [7, 300, 1500, 4000]
    q, kp, vp, table, lt = _nhd_case(lens, 16, dtype, seed=max_seq_len % 97)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=max_seq_len, scale=128 ** -0.5)
    ref = oracle.paged_decode(q, kp, vp, table, lt, 128 ** -0.5)
    assert _err(out, ref) <= (TOL if dtype != torch.float32 else 1e-5)


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("cumulative", [False, True])
def test_early_issue_one_partition_per_pair(dev, idx_dtype, cumulative):
    # 40 sequences x 8 kv heads = 320 pairs, more than the CUs: one partition per
    # pair, so each wave requests its first tiles before the context length has
    # arrived.  Zero-length contexts, contexts shorter than one tile, unmapped
    # blocks (-1 and past num_blocks) inside the early tiles, the fused write of
    # the current row, and int32/int64 tables, lengths and slots.
    lens = [0, 1, 15, 16, 17, 33, 600, 0, 250, 129] * 4
    bs = 16
    q, kp, vp, table, _ = _nhd_case(lens, bs, torch.bfloat16, seed=77)
    nb = kp.shape[0]
    keep = torch.ones(len(lens), max(lens), dtype=torch.bool)
    table[6, 1] = -1            # tokens 16..31 of a 600-token context
    keep[6, 16:32] = False
    table[8, 0] = nb + 5        # tokens 0..15 of a 250-token context
    keep[8, 0:16] = False
    g = torch.Generator().manual_seed(78)
    nk = (torch.randn(len(lens), 8, 128, generator=g) * 0.5).to(torch.bfloat16)
    nv = (torch.randn(len(lens), 8, 128, generator=g) * 0.5).to(torch.bfloat16)
    slots = torch.tensor([int(table[b, (n - 1) // bs]) * bs + (n - 1) % bs if n > 0 else -1
                          for b, n in enumerate(lens)], dtype=idx_dtype)
    lt = torch.tensor(lens, dtype=idx_dtype)
    if cumulative:
        lt = torch.cat([torch.zeros(1, dtype=idx_dtype), torch.cumsum(lt, 0).to(idx_dtype)])
    kd, vd = kp.to(dev), vp.to(dev)
    out = ops.paged_decode(q.to(dev), kd, vd, table.to(idx_dtype).to(dev), lt.to(dev),
                           lens_cumulative=cumulative, max_seq_len=max(lens),
                           scale=128 ** -0.5, new_k=nk.to(dev), new_v=nv.to(dev),
                           new_slots=slots.to(dev)).cpu()
    ek, ev = oracle.store_kvcache(nk, nv, kp, vp, slots.long())
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    assert torch.count_nonzero(out[[0, 7, 10, 17]]) == 0
    safe = table.clone()
    safe[6, 1] = 0
    safe[8, 0] = 0
    ref = oracle.paged_decode(q, ek, ev, safe, torch.tensor(lens), 128 ** -0.5, valid_mask=keep)
    live = [b for b, n in enumerate(lens) if n > 0]
    assert _err(out[live], ref[live]) <= TOL


@pytest.mark.parametrize("B", [3, 40])
@pytest.mark.parametrize("width,shift", [(704, 0), (300, 0), (601, 0), (704, 3), (20001, 1)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_key_valid_mask_on_matrix_cores(dev, B, width, shift, dtype):
    # The TTS decode's key_valid_mask on the matrix-core kernel: B=3 splits
    # contexts into partitions, B=40 runs one partition per pair with the early
    # tile requests.  Widths: past every context (704), shorter than some
    # contexts (300: later tokens count as valid), and odd (601: rows start
    # at every byte offset within a 4-byte word), and wider than 16 KiB.
    # shift places the whole mask at a storage offset of that many bytes.  One
    # sequence has every token masked and must come out 0.
    base = [1, 15, 16, 17, 130, 299, 300, 301, 600, 700]
    lens = (base * ((B + len(base) - 1) // len(base)))[:B]
    q, kp, vp, table, lt = _nhd_case(lens, 16, dtype, seed=B + width)
    g = torch.Generator().manual_seed(width)
    valid = torch.rand(B, width, generator=g) < 0.8
    dead = 1 if B > 1 else 0
    valid[dead] = False
    flat = torch.zeros(shift + B * width, dtype=torch.bool, device=dev)
    flat[shift:] = valid.flatten().to(dev)
    vdev = flat[shift:].view(B, width)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=max(lens), scale=128 ** -0.5, valid_mask=vdev).cpu()
    ref = oracle.paged_decode(q, kp, vp, table, lt, 128 ** -0.5, valid_mask=valid)
    if lens[dead] <= width:
        assert torch.count_nonzero(out[dead]) == 0
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_key_valid_mask_past_64_tiles_per_wave(dev, dtype):
    # One partition per pair (40 sequences) and a 9100-token context: its
    # waves hold the block ids and mask bits of 64 tiles at a time and reload
    # both for tiles 64 onwards.
    lens = [9100] + [40 + 7 * i for i in range(39)]
    q, kp, vp, table, lt = _nhd_case(lens, 16, dtype, seed=91)
    g = torch.Generator().manual_seed(92)
    valid = torch.rand(len(lens), 9105, generator=g) < 0.7
    valid[0, 8192:8200] = False  # a run of masked tokens past the 64th tile of a wave
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=max(lens), scale=128 ** -0.5,
                           valid_mask=valid.to(dev)).cpu()
    ref = oracle.paged_decode(q, kp, vp, table, lt, 128 ** -0.5, valid_mask=valid)
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv,B,split", [(16, 8, 32, 0), (16, 8, 48, 0), (16, 8, 20, 256),
                                           (8, 1, 300, 0)])
def test_four_wave_workgroups_with_prologue_mask_and_store(dev, dtype, hq, hkv, B, split):
    # 16-bit pools at head_dim 128 take four-wave workgroups when a launch has
    # more workgroups than CUs (B = 48 x 8 kv heads; 20 x 8 in partitions of
    # 256 tokens, merged; 300 sequences of one kv head), eight waves at one per
    # CU (32 x 8).  With the fused prologue, the key mask and the fused store:
    # bit for bit the two-launch path (va_qk_norm_rope, then the decode), output
    # and pools, and the oracle within the tolerance.  (The prologue's sum of
    # squares is reduced in another order than the oracle's mean, so the stored
    # keys may differ from the oracle's by an ulp.)
    g = torch.Generator().manual_seed(B + hq)
    lens = torch.randint(1, 700, (B,), generator=g).tolist()
    q, kp, vp, table, lt = _nhd_case(lens, 16, dtype, hq=hq, hkv=hkv, seed=B)
    nk = torch.randn(B, hkv, 128, generator=g).to(dtype)
    nv = torch.randn(B, hkv, 128, generator=g).to(dtype)
    wq = (torch.rand(128, generator=g) + 0.5).to(dtype)
    wk = (torch.rand(128, generator=g) + 0.5).to(dtype)
    cs = oracle.rope_cache(128, 1024, 1_000_000.0)
    pos = lt.long() - 1
    valid = torch.rand(B, max(lens) + 5, generator=g) < 0.85
    print(f"four-wave case {dtype} hq={hq} hkv={hkv} B={B} split={split}", flush=True)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    common = dict(max_seq_len=max(lens), scale=128 ** -0.5, split_tokens=split,
                  valid_mask=valid.to(dev), new_v=nv.to(dev))
    td, ld = table.to(dev), lt.to(dev)
    kd1, vd1 = kp.to(dev), vp.to(dev)
    kd2, vd2 = kd1.clone(), vd1.clone()
    out1 = ops.paged_decode(q.to(dev), kd1, vd1, td, ld, new_k=nk.to(dev), prologue=pro,
                            **common)
    qn, kn = ops.qk_norm_rope(q.to(dev), nk.to(dev), pro)
    out2 = ops.paged_decode(qn, kd2, vd2, td, ld, new_k=kn, **common)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(kd1, kd2) and torch.equal(vd1, vd2)
    rq, rk = oracle.qk_norm_rope(q, nk, pos, wq, wk, 1e-6, cs)
    ek, ev = oracle.write_current_kv(kp, vp, table, lt, rk, nv, layout=ops.LAYOUT_NHD)
    assert torch.equal(vd1.cpu(), ev)
    ref = oracle.paged_decode(rq, ek, ev, table, lt, 128 ** -0.5, valid_mask=valid)
    assert _err(out1, ref) <= TOL
