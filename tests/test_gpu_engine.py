"""Mini engine on the GPU: a stack of PagedAttention layers driven by the
metadata producers the way the engine drives them.  An eager prefill is
followed by decode steps run twice: eagerly (ModelRunner._prepare) and as
HIP-graph replays over static padded buffers (GraphRunner.run).  The
reference gates graph mode on equality with eager
(tests/test_cuda_graph.py:99-142); here the outputs and the caches must match
bit for bit, and layer 0's cache rows must equal the projected k/v rows."""

from dataclasses import dataclass, field

import pytest
import torch
from torch import nn

from voiceagent_amd.engine import DecodeGraphMetadata, prepare_batch
from voiceagent_amd.layers.attention import PagedAttention
from voiceagent_amd.layers.context import attention_context
from voiceagent_amd.layers.qwen3 import Qwen3AttentionCore

pytestmark = pytest.mark.gpu

L, HQ, HKV, D, BS, HID = 4, 16, 8, 128, 16, 256
NB = 64
MAX_MODEL_LEN = 256


@dataclass
class Seq:
    length: int
    num_computed_tokens: int = 0
    block_table: list[int] = field(default_factory=list)

    def __len__(self):
        return self.length


class TinyDecoder(nn.Module):
    """Attention-only decoder: x += o_proj(attn(split(x @ Wqkv))) per layer, with
    the engine's fused-qkv views (v strided by (Hq + 2 Hkv) D).  ``kind``
    "paged" uses PagedAttention on the raw q/k; "qwen3" uses
    Qwen3AttentionCore (q/k RMSNorm + RoPE at the token positions first)."""

    def __init__(self, dev, seed, kind="paged"):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.wqkv = [(torch.randn(HID, (HQ + 2 * HKV) * D, generator=g) * HID ** -0.5)
                     .to(torch.bfloat16).to(dev) for _ in range(L)]
        self.wo = [(torch.randn(HQ * D, HID, generator=g) * (HQ * D) ** -0.5)
                   .to(torch.bfloat16).to(dev) for _ in range(L)]
        self.kind = kind
        if kind == "paged":
            self.attn = nn.ModuleList(PagedAttention(HQ, D, D ** -0.5, HKV) for _ in range(L))
        else:
            self.attn = nn.ModuleList(
                Qwen3AttentionCore(HQ, D, HKV, eps=1e-6, max_position=MAX_MODEL_LEN)
                for _ in range(L))
            for layer in self.attn:
                layer.q_norm_weight.data = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
                layer.k_norm_weight.data = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
            self.attn.to(dev)
        kv = torch.zeros(2, L, NB, BS, HKV, D, dtype=torch.bfloat16, device=dev)
        self.kv = kv
        for i, layer in enumerate(self.attn):  # model_runner.py:116-131
            layer.k_cache = kv[0, i]
            layer.v_cache = kv[1, i]
        self.record = None  # list collecting layer 0's (k, v) rows when set

    def forward(self, x, positions):
        for i in range(L):
            qkv = x @ self.wqkv[i]
            q, k, v = qkv.split([HQ * D, HKV * D, HKV * D], dim=-1)
            if i == 0 and self.record is not None:
                self.record.append((k.reshape(-1, HKV, D).clone(), v.reshape(-1, HKV, D).clone()))
            q, k, v = q.view(-1, HQ, D), k.view(-1, HKV, D), v.view(-1, HKV, D)
            if self.kind == "paged":
                a = self.attn[i](q, k, v)
            else:
                a = self.attn[i](positions, q, k, v)
            x = x + a.flatten(1) @ self.wo[i]
        return x


def _sequences(prompts, seed):
    g = torch.Generator().manual_seed(seed)
    free = (torch.randperm(NB - 1, generator=g) + 1).tolist()  # block 0 stays free
    seqs = []
    for n in prompts:
        nblk = (n + 8 + BS - 1) // BS  # room for the decode steps
        seqs.append(Seq(n, 0, [free.pop() for _ in range(nblk)]))
    return seqs


@pytest.mark.parametrize("kind", ["paged", "qwen3"])
def test_eager_and_graph_decode_match(dev, kind):
    prompts = [37, 5, 64, 17, 100, 1]
    steps = 3
    g = torch.Generator().manual_seed(3)
    emb = [torch.randn(MAX_MODEL_LEN, HID, generator=g).to(torch.bfloat16).to(dev)
           for _ in prompts]
    engines = {}
    modes = ("eager", "graph") + (("unfused",) if kind == "qwen3" else ())
    for mode in modes:
        model = TinyDecoder(dev, seed=1, kind=kind)
        if mode == "eager":
            model.record = []
        if mode == "unfused":  # prologue kernel + decode: two launches per layer
            for layer in model.attn:
                layer.fuse_prologue = False
        seqs = _sequences(prompts, seed=2)
        positions, ctx = prepare_batch(seqs, BS, dev)
        with attention_context(ctx):
            model(torch.cat([emb[i][: len(s)] for i, s in enumerate(seqs)]), positions)
        for s in seqs:
            s.num_computed_tokens = len(s)
        engines[mode] = (model, seqs)

    # Graph mode: capture one bucket over static buffers (graph_runner.py:96-138).
    model_g, seqs_g = engines["graph"]
    meta = DecodeGraphMetadata(max_batch_size=8, max_blocks=16, block_size=BS,
                               max_model_len=MAX_MODEL_LEN, device=dev, buckets=[8])
    x_static = torch.zeros(8, HID, dtype=torch.bfloat16, device=dev)
    meta.warmup_state()
    ctx_g = meta.context(8)
    pos_g = meta.positions[:8]
    with attention_context(ctx_g):
        for _ in range(2):
            model_g(x_static, pos_g)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out_static = model_g(x_static, pos_g)
    torch.cuda.synchronize()
    # The warm-up and the capture wrote nothing (every slot was -1).
    model_e, seqs_e = engines["eager"]
    assert torch.equal(model_g.kv, model_e.kv)

    for step in range(steps):
        for _, seqs in engines.values():
            for s in seqs:
                s.length += 1
                s.num_computed_tokens = s.length - 1
        x = torch.stack([emb[i][len(s) - 1] for i, s in enumerate(seqs_e)])
        positions, ctx = prepare_batch(seqs_e, BS, dev)
        with attention_context(ctx):
            out_e = model_e(x, positions)
        if "unfused" in engines:
            model_u, seqs_u = engines["unfused"]
            positions_u, ctx_u = prepare_batch(seqs_u, BS, dev)
            with attention_context(ctx_u):
                out_u = model_u(x, positions_u)
            assert torch.equal(out_e, out_u), step
        bucket = meta.stage(seqs_g)
        assert bucket == 8
        x_static.zero_()
        x_static[: len(seqs_g)].copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        out_g = out_static[: len(seqs_g)]
        print(f"step {step}: max |eager - graph| = {(out_e - out_g).abs().max().item()}",
              flush=True)
        assert torch.equal(out_e, out_g), step

    assert torch.equal(model_g.kv, model_e.kv)
    if "unfused" in engines:
        assert torch.equal(engines["unfused"][0].kv, model_e.kv)
    if kind == "qwen3":
        return  # layer 0's cache holds normalised, rotated keys: covered by test_gpu_prologue

    # Every slot written in layer 0 holds exactly the k/v row the layer
    # produced for that (sequence, position), bit for bit.
    rec = model_e.record
    assert len(rec) == 1 + steps
    rows = {}
    t = 0
    for i, n in enumerate(prompts):  # prefill rows, packed in sequence order
        for p in range(n):
            rows[(i, p)] = (rec[0][0][t], rec[0][1][t])
            t += 1
    for step in range(steps):  # one decode row per sequence per step
        for i, n in enumerate(prompts):
            rows[(i, n + step)] = (rec[1 + step][0][i], rec[1 + step][1][i])
    for (i, p), (k, v) in rows.items():
        s = seqs_e[i]
        blk, off = s.block_table[p // BS], p % BS
        assert torch.equal(model_e.kv[0, 0, blk, off], k), (i, p)
        assert torch.equal(model_e.kv[1, 0, blk, off], v), (i, p)
