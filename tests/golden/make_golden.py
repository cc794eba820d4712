"""Regenerate the golden fixtures under tests/golden/ (run from the repo root).

tts_seed17.npz  — the seeded fixture of the reference's TTS kernel tests
                  (tests/test_qwen_tts_paged_attention_kernel.py:16-35: seed 17,
                  pages (3, 5, 1, 7, 2) drawn in that order, q = ones, tables
                  [[3,5,0],[1,7,2]], seq_lens [3,5], left-padded valid mask),
                  the new K/V rows drawn next from the same RNG stream (:146-147),
                  and the float64 brute-force outputs with and without the
                  fused current-row write.
cfg1_decode.npz — config 1 (4 sequences, fp32 N(0,1), pool [128,16,8,128], seed 0):
                  input checksums and the float64 brute-force output.

Inputs are regenerated with torch's CPU generator; expected outputs come
from tests/golden/brute.py (scalar loops), never from the oracle.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from tests.golden import brute  # noqa: E402
from voiceagent_amd import workloads  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def tts_seed17_inputs():
    page_table = torch.tensor([[3, 5, 0], [1, 7, 2]], dtype=torch.long)
    seq_lens = torch.tensor([3, 5], dtype=torch.long)
    valid = torch.tensor(
        [[True, True, True, False, False], [False, True, True, True, True]], dtype=torch.bool
    )
    k_pool = torch.zeros((8, 2, 2, 4), dtype=torch.float32)
    v_pool = torch.zeros_like(k_pool)
    torch.manual_seed(17)
    for page in (3, 5, 1, 7, 2):
        k_pool[page].normal_()
        v_pool[page].normal_()
    q = torch.ones((2, 4, 1, 4), dtype=torch.float32)
    new_key = torch.randn((2, 2, 1, 4), dtype=torch.float32)
    new_value = torch.randn((2, 2, 1, 4), dtype=torch.float32)
    return q, k_pool, v_pool, page_table, seq_lens, valid, new_key, new_value


def make_tts_seed17():
    q, kp, vp, table, lens, valid, nk, nv = tts_seed17_inputs()
    scale = 0.5  # 1 / sqrt(4)
    out = brute.paged_decode(q[:, :, 0].tolist(), kp.tolist(), vp.tolist(), table.tolist(),
                             lens.tolist(), scale, layout="hnd", valid=valid.tolist())
    kp2, vp2 = kp.clone(), vp.clone()
    for row in range(2):
        pos = int(lens[row]) - 1
        page, off = int(table[row, pos // 2]), pos % 2
        kp2[page, :, off] = nk[row, :, 0]
        vp2[page, :, off] = nv[row, :, 0]
    out_fused = brute.paged_decode(q[:, :, 0].tolist(), kp2.tolist(), vp2.tolist(),
                                   table.tolist(), lens.tolist(), scale, layout="hnd",
                                   valid=valid.tolist())
    np.savez(
        os.path.join(HERE, "tts_seed17.npz"),
        q=q.numpy(), k_pool=kp.numpy(), v_pool=vp.numpy(), page_table=table.numpy(),
        seq_lens=lens.numpy(), valid=valid.numpy(), new_key=nk.numpy(), new_value=nv.numpy(),
        expected=np.array(out, dtype=np.float64),
        expected_fused=np.array(out_fused, dtype=np.float64),
        k_pool_fused=kp2.numpy(), v_pool_fused=vp2.numpy(),
    )


def make_cfg1():
    lens = workloads.cfg1_lens(0)
    b = workloads.make_decode_batch(lens, num_blocks=128, dtype=torch.float32, seed=0)
    out = brute.paged_decode(b.q.tolist(), b.k_pools[0].tolist(), b.v_pools[0].tolist(),
                             b.block_tables.tolist(), lens, b.scale, layout="nhd")
    np.savez(
        os.path.join(HERE, "cfg1_decode.npz"),
        lens=np.array(lens), block_tables=b.block_tables.numpy(),
        q_sum=np.float64(b.q.double().sum()), k_sum=np.float64(b.k_pools[0].double().sum()),
        v_sum=np.float64(b.v_pools[0].double().sum()),
        expected=np.array(out, dtype=np.float64),
    )


if __name__ == "__main__":
    make_tts_seed17()
    make_cfg1()
    print("golden fixtures written to", HERE)
