"""The engine's decode-graph set on the GPU, as GraphRunner captures it
(qwen_asr_vllm/engine/graph_runner.py:32, 97-191): buckets
(1, 2, 4, 8, 16, 24, 32, 48, 64) captured largest first into one shared
memory pool, on torch's own capture stream, with max_seqlen_k baked at
max_model_len = 65536.  At that bound every bucket up to 16 runs the
length-dependent context split plus the merge kernel inside its graph, and
the decode workspace is allocated during the capture.

Each replay (real lengths, padded rows up to the bucket, contexts past 4096
tokens) is checked against the CPU oracle (store + decode, pools bit-exact,
outputs max-abs 2e-2 in bf16) and against an eager launch with the same
context (bit-exact), after tests/test_cuda_graph.py:99-142, which gates graph
mode on equality with eager.  No workspace a graph holds may be freed.
"""

import math

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops
from voiceagent_amd.engine import DecodeGraphMetadata
from voiceagent_amd.layers.attention import PagedAttention
from voiceagent_amd.layers.context import attention_context

pytestmark = pytest.mark.gpu

BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64)  # graph_runner.py:32
MAX_MODEL_LEN = 65536
HQ, HKV, D, BS, LAYERS = 16, 8, 128, 16, 2
NB = 4800
MAX_BLOCKS = 320  # 5120 tokens per sequence


class Seq:
    """The three attributes the graph staging reads (graph_runner.py:163-176)."""

    def __init__(self, length, block_table):
        self.length = length
        self.num_computed_tokens = length - 1
        self.block_table = block_table

    def __len__(self):
        return self.length


def test_bucket_set_captured_largest_first_replays_match_oracle_and_eager(dev):
    gen = torch.Generator().manual_seed(2024)
    kv = (torch.randn(2, LAYERS, NB, BS, HKV, D, generator=gen) * 0.5).to(torch.bfloat16).to(dev)
    layers = [PagedAttention(HQ, D, D ** -0.5, HKV) for _ in range(LAYERS)]
    for i, layer in enumerate(layers):  # model_runner.py:116-131
        layer.k_cache, layer.v_cache = kv[0, i], kv[1, i]
    q_st = torch.zeros(LAYERS, 64, HQ, D, dtype=torch.bfloat16, device=dev)
    k_st = torch.zeros(LAYERS, 64, HKV, D, dtype=torch.bfloat16, device=dev)
    v_st = torch.zeros(LAYERS, 64, HKV, D, dtype=torch.bfloat16, device=dev)

    def forward(n):
        return [layers[i](q_st[i, :n], k_st[i, :n], v_st[i, :n]) for i in range(LAYERS)]

    meta = DecodeGraphMetadata(max_batch_size=64, max_blocks=MAX_BLOCKS, block_size=BS,
                               max_model_len=MAX_MODEL_LEN, device=dev, buckets=BUCKETS)
    meta.warmup_state()
    retired_before = len(ops._RETIRED)
    graphs, outs, pool = {}, {}, None
    for n in reversed(BUCKETS):  # graph_runner.py:116-137
        print(f"capture bucket {n}", flush=True)
        with attention_context(meta.context(n)):
            for _ in range(2):
                forward(n)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool):
                outs[n] = forward(n)
        pool = pool or graph.pool()
        graphs[n] = graph
    torch.cuda.synchronize()
    # The split buckets took their workspace during capture, on the capture
    # stream; nothing was replaced (and so nothing a graph holds was dropped).
    assert len(ops._RETIRED) == retired_before
    cap_key = (dev.index or 0, torch.cuda.graphs.graph.default_capture_stream.cuda_stream)
    assert cap_key in ops._WORKSPACES
    assert ops._WORKSPACES[cap_key].numel() >= ops.decode_workspace_bound(dev, HQ, HKV, D)

    free = torch.randperm(NB - 1, generator=gen).add(1).tolist()  # block 0 stays padding
    # (batch size, lengths): padded buckets, and contexts past 4096 tokens.
    steps = [(1, [4500]), (2, [4097, 33]), (3, [1, 700, 5100]), (7, None), (13, None),
             (16, None), (1, [17]), (16, None), (5, [4096, 4095, 1, 2, 3000])]
    for step, (batch, lens) in enumerate(steps):
        if lens is None:
            lens = torch.randint(1, 5120, (batch,), generator=gen).tolist()
            lens[0] = max(lens[0], 4200)
        seqs = []
        cursor = 0
        for n in lens:
            need = math.ceil(n / BS)
            seqs.append(Seq(n, free[cursor:cursor + need]))
            cursor += need
        bucket = meta.stage(seqs)
        assert bucket == next(b for b in BUCKETS if b >= batch)
        q = torch.randn(LAYERS, batch, HQ, D, generator=gen).to(torch.bfloat16)
        k = (torch.randn(LAYERS, batch, HKV, D, generator=gen) * 0.5).to(torch.bfloat16)
        v = (torch.randn(LAYERS, batch, HKV, D, generator=gen) * 0.5).to(torch.bfloat16)
        for t, src in ((q_st, q), (k_st, k), (v_st, v)):
            t.zero_()
            t[:, :batch].copy_(src)
        pools_before = kv.cpu()
        print(f"replay step {step}: batch {batch} bucket {bucket} lens {lens}", flush=True)
        graphs[bucket].replay()
        torch.cuda.synchronize()
        got = [o[:batch].clone() for o in outs[bucket]]
        pools_after = kv.cpu()
        # Padding rows [batch, bucket) (slot -1, table 0, k_len 1;
        # graph_runner.py:157-160, 178-180) are discarded by the caller but
        # must be finite.
        for i in range(LAYERS):
            pad = outs[bucket][i][batch:bucket]
            assert pad.shape[0] == bucket - batch
            assert bool(torch.isfinite(pad).all()), (step, i, "non-finite padding row")

        # Oracle: the store of every real row, then the decode over the pool.
        slots = meta.slot_mapping[:batch].cpu()
        table = meta.block_tables[:batch].cpu()
        lens_t = torch.tensor(lens)
        for i in range(LAYERS):
            ek, ev = oracle.store_kvcache(k[i], v[i], pools_before[0, i], pools_before[1, i], slots)
            assert torch.equal(pools_after[0, i], ek) and torch.equal(pools_after[1, i], ev), \
                (step, i)
            ref = oracle.paged_decode(q[i], ek, ev, table, lens_t, D ** -0.5)
            err = (got[i].float().cpu() - ref).abs().max().item()
            print(f"  layer {i}: max-abs error vs oracle {err:.3e}", flush=True)
            assert err <= 2e-2, (step, i)

        # Eager with the graph's own context (max_seqlen_k = max_model_len):
        # the same launches, so the same bits.  Re-storing the same rows to
        # the same slots leaves the pools unchanged.
        with attention_context(meta.context(bucket)):
            eager = [o[:batch] for o in forward(bucket)]
        torch.cuda.synchronize()
        for i in range(LAYERS):
            assert torch.equal(eager[i], got[i]), (step, i)
        assert torch.equal(kv.cpu(), pools_after)
