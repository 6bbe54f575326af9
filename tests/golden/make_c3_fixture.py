"""Writes tests/golden/c3_check.npz: host outputs of the C3 workload (the
1B-class SAF model: 24 layers, d_model 2048, 16 heads, hd 128, B=2, T=8192,
four dense-pattern heads per layer), computed by the fp32 oracle
(oracle/model_oracle.py, the reference's CPU split path).

The model is bench.py's C3 build made on the CPU (seed-1337 weights rounded
to bf16 as on the GPU, CPU-seeded pattern logits, the same bf16 compact
patterns).  Stored: the last-position logits of both sequences and the final
LayerNorm outputs at sampled positions.  bench.py (c3) and
tests/test_gpu_configs.py compare the GPU prefill with them.  Run from the
repository root on the CPU (several minutes, about 30 GB of memory):

    python tests/golden/make_c3_fixture.py
"""
import hashlib
import os
import sys
import time

import numpy as np
import torch
import torch.nn.functional as F

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(REPO, "selective-attention-freezing_amd"), REPO]

import bench  # noqa: E402
from oracle import model_oracle  # noqa: E402

OUT = os.path.join(REPO, "tests", "golden", "c3_check.npz")
T, L = 8192, 24
POSITIONS = [0, 1, 63, 64, 255, 1000, 4095, 4096, 6000, T - 1]


def main():
    torch.set_num_threads(os.cpu_count())
    t0 = time.time()
    m, x, plan = bench.build_c3_model(T, L, "cpu")
    print(f"model built in {time.time() - t0:.0f} s", flush=True)
    cfg = m.config
    sd = {k: v.detach().float() for k, v in m.state_dict().items() if not k.endswith("dyn_pattern")}
    freeze = []
    for blk in m.transformer.h:
        a = blk.attn
        rec = {"frozen": a.dyn_frozen.tolist(), "patterns": {}, "decomp": {}}
        for h in range(cfg.n_head):
            if rec["frozen"][h]:
                rec["patterns"][h] = a.dyn_pattern[int(a.dyn_pattern_slot[h])]   # bf16, widened per head
        freeze.append(rec)
    ocfg = {"n_layer": cfg.n_layer, "n_head": cfg.n_head, "n_embd": cfg.n_embd,
            "position_encoding": "rope", "rope_base": cfg.rope_base}
    hidden = model_oracle.gpt_forward(sd, ocfg, freeze, x, path="split", positions=POSITIONS, head=False)
    logits = F.linear(hidden[:, -1], sd["lm_head.weight"])
    tok_hash = hashlib.sha256(x.numpy().astype(np.int64).tobytes()).hexdigest()
    np.savez_compressed(OUT, logits_last=logits.numpy().astype(np.float32),
                        hidden=hidden.numpy().astype(np.float32), positions=np.array(POSITIONS),
                        tokens_sha256=np.array(tok_hash), plan=np.array(repr(sorted(plan.items()))),
                        T=np.array(T), L=np.array(L))
    print(f"wrote {OUT} in {time.time() - t0:.0f} s; |logits| max {logits.abs().max():.3f}", flush=True)


if __name__ == "__main__":
    main()
