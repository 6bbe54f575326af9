"""Writes tests/golden/c4_check.npz: host outputs of the C4 workload (Qwen3-
style GQA backbone: 24 layers, hidden 896, 14 query / 2 KV heads, hd 64,
RoPE theta 1e6, B=4, T=4096) with round(r * 14) query heads per layer frozen
to the causal mean for r = 0.25, 0.5, 0.75 (f = 4, 7, 10), computed by the
fp32 oracle (oracle/qwen_oracle.py, the reference's hybrid split path).

The model is bench.py's C4 build made on the CPU (qwen.build_model: seed-1337
transformers init on the CPU, cast to bf16; the frozen sets of
qwen.nested_head_masks; seeded tokens).  The oracle rotates with the bf16
model's own RoPE frequencies: transformers casts the rotary inv_freq buffer
along with the weights, so a bf16 model (and the same model cast back to
fp32) uses bf16-rounded frequencies.  Stored per f (0, 4, 7, 10): the
final-norm hidden states at sampled positions of all four sequences, and the
cosine that the same model reaches against them when it runs in bf16 through
torch alone on the CPU (transformers' modules and the hybrid adapter's
torch split path): the bf16 level of this 24-layer random-init model, which
no bf16 forward of it improves on (transformers' own bf16 forward reaches
0.9997 at f = 0).  bench.py (c4) and tests/test_gpu_configs.py compare the
GPU prefill with them.  Run from the repository root on the CPU (several
minutes, about 15 GB of memory):

    python tests/golden/make_c4_fixture.py
"""
import hashlib
import os
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(REPO, "selective-attention-freezing_amd"), REPO]

import qwen  # noqa: E402
from oracle import qwen_oracle  # noqa: E402

OUT = os.path.join(REPO, "tests", "golden", "c4_check.npz")
B, T, L = 4, 4096, 24
RATES = (0.0, 0.25, 0.5, 0.75)
POSITIONS = [0, 1, 63, 64, 255, 1000, 2047, 2048, 3000, T - 1]


def _cos(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    return float(a @ b / (a.norm() * b.norm()))


def main():
    torch.set_num_threads(os.cpu_count())
    t0 = time.time()
    cfg = qwen.qwen_config(n_layers=L, max_positions=max(T, 4096))
    model = qwen.build_model(cfg, device="cpu", dtype=torch.bfloat16, seed=1337)
    sd = {k: v.detach().float() for k, v in model.state_dict().items() if not k.startswith("lm_head")}
    inv_freq = model.model.rotary_emb.inv_freq.float().clone()
    del model
    ids = torch.randint(0, 151643, (B, T), generator=torch.Generator().manual_seed(1337))
    H = cfg.num_attention_heads
    ocfg = dict(n_layers=L, n_heads=H, n_kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                eps=cfg.rms_norm_eps, rope_theta=1e6)
    mean = torch.ones(T, T).tril_().expand(H, T, T)
    out = {"positions": np.array(POSITIONS), "T": np.array(T), "L": np.array(L), "B": np.array(B),
           "tokens_sha256": np.array(hashlib.sha256(ids.numpy().astype(np.int64).tobytes()).hexdigest())}
    for rate in RATES:
        masks = qwen.nested_head_masks(rate, L, H)
        f = int(masks[0].sum())
        fr = [{"mask": m.numpy(), "dense": mean} for m in masks] if f else None
        hid = qwen_oracle.qwen_forward(sd, ocfg, fr, ids, inv_freq=inv_freq)[:, POSITIONS]
        out[f"hidden_f{f}"] = hid.numpy().astype(np.float32)
        # the same model in bf16 through torch alone (adapter split path on the CPU)
        model = qwen.build_model(cfg, device="cpu", dtype=torch.bfloat16, seed=1337)
        if f:
            qwen.convert_with_rate(model, rate, T)
        with torch.no_grad():
            got = qwen.backbone_forward(model.model, ids)[:, POSITIONS].float()
        del model
        out[f"bf16_cos_f{f}"] = np.array(_cos(got, hid))
        print(f"f={f} done at {time.time() - t0:.0f} s; torch bf16 cosine {float(out[f'bf16_cos_f{f}']):.7f}",
              flush=True)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} in {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main()
