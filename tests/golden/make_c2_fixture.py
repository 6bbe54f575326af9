"""Writes tests/golden/c2_last_logits.npz: the last-position logits of the C2
headline workload, computed by the fp32 oracle (oracle/model_oracle.py, the
reference's CPU split path) on the host.

The model is bench.py's C2 build (124M nanoGPT, seed-1337 random init on the
CPU, 36/144 heads frozen to mean / decay / window, T = 16384, seeded tokens),
with its weights rounded to bf16 as on the GPU.  bench.py compares the GPU
prefill output with these logits (cosine) before it times anything.  Run from
the repository root on the CPU (about 2 minutes, 12 GB of memory):

    python tests/golden/make_c2_fixture.py
"""
import hashlib
import os
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(REPO, "selective-attention-freezing_amd"), REPO]

import bench  # noqa: E402
from oracle import model_oracle  # noqa: E402

OUT = os.path.join(REPO, "tests", "golden", "c2_last_logits.npz")


def oracle_inputs(m):
    cfg = m.config
    sd = {k: v.detach().float().cpu() for k, v in m.state_dict().items()}
    freeze = []
    for blk in m.transformer.h:
        a = blk.attn
        rec = {"frozen": a.dyn_frozen.cpu().tolist(), "patterns": {}, "decomp": {}}
        for h in range(cfg.n_head):
            if rec["frozen"][h]:
                rec["decomp"][h] = (a.dyn_alpha[h].cpu(), a.dyn_rho[h].cpu(), a.dyn_z[h].cpu())
        freeze.append(rec)
    ocfg = {"n_layer": cfg.n_layer, "n_head": cfg.n_head, "n_embd": cfg.n_embd,
            "position_encoding": "rope", "rope_base": cfg.rope_base}
    return sd, ocfg, freeze


def main():
    T = 16384
    t0 = time.time()
    m, x, plan = bench.build_c2_model(T, "cpu", torch.bfloat16)
    sd, ocfg, freeze = oracle_inputs(m)
    del m
    logits = model_oracle.gpt_forward(sd, ocfg, freeze, x, path="split")[0, -1].numpy()
    tok_hash = hashlib.sha256(x.numpy().astype(np.int64).tobytes()).hexdigest()
    kinds = [(int(l), int(h), k, float(p)) for l, hs in sorted(plan.items()) for h, k, p in hs]
    np.savez_compressed(OUT, logits=logits.astype(np.float32), tokens_sha256=np.array(tok_hash),
                        plan=np.array(repr(kinds)), T=np.array(T))
    print(f"wrote {OUT} in {time.time() - t0:.0f} s; |logits| max {np.abs(logits).max():.3f}")


if __name__ == "__main__":
    main()
