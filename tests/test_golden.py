"""Golden vectors written from the reference's own CPU code
(tests/golden/make_golden.py): a 3-layer, 2-head RoPE GPT with a dense-frozen
head, a generic decomposed head and a causal-mean head.

CPU: the oracle's model restatement reproduces the reference's split-path and
eager-path logits, and the oracle's pattern helpers reproduce the stored
decomposed buffers and rho band.  GPU: the bf16 HIP model loaded with the same
weights and freeze state reproduces them with logits cosine >= 0.9999.
"""
import os

import numpy as np
import pytest
import torch

from oracle import model_oracle, saf_oracle as orc

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gpt_forward_small.npz")


def _load():
    d = np.load(FIX, allow_pickle=False)
    n_layer, n_head, n_embd, vocab, block = (int(x) for x in d["cfg"])
    sd = {k[2:]: torch.from_numpy(d[k].astype(np.float32)) for k in d.files if k.startswith("w:")}
    freeze = []
    for l in range(n_layer):
        fr = d[f"frozen:{l}"]
        dec = d[f"decomp:{l}"]
        rec = {"frozen": fr.tolist(), "patterns": {}, "decomp": {}}
        for h in range(n_head):
            if fr[h] and dec[h]:
                rec["decomp"][h] = tuple(torch.from_numpy(d[f"{n}:{l}"][h]) for n in ("alpha", "rho", "z"))
            elif fr[h]:
                rec["patterns"][h] = torch.from_numpy(d[f"pattern:{l}"][h])
        freeze.append(rec)
    cfg = {"n_layer": n_layer, "n_head": n_head, "n_embd": n_embd, "position_encoding": "rope",
           "rope_base": 10000.0, "vocab": vocab, "block": block}
    return d, sd, cfg, freeze


def test_oracle_model_matches_reference_split_path():
    d, sd, cfg, freeze = _load()
    x = torch.from_numpy(d["tokens"])
    got = model_oracle.gpt_forward(sd, cfg, freeze, x, path="split", all_positions=True)
    np.testing.assert_allclose(got.numpy(), d["logits_split"], atol=2e-5, rtol=1e-5)


def test_oracle_model_matches_reference_eager_path():
    d, sd, cfg, freeze = _load()
    x = torch.from_numpy(d["tokens"])
    got = model_oracle.gpt_forward(sd, cfg, freeze, x, path="eager", all_positions=True)
    np.testing.assert_allclose(got.numpy(), d["logits_eager"], atol=2e-5, rtol=1e-5)


def test_decomposed_storage_and_band_match_reference():
    d, _, cfg, _ = _load()
    for l in range(cfg["n_layer"]):
        key = f"rho_band:{l}"
        if key not in d.files:
            continue
        rho = d[f"rho:{l}"]
        dec = d[f"decomp:{l}"]
        band = orc.make_rho_band(rho)
        for h in np.nonzero(dec)[0]:
            np.testing.assert_array_equal(band[h], d[key][h])
            z = orc.decomposed_logz(d[f"alpha:{l}"][h:h + 1], rho[h:h + 1])[0]
            np.testing.assert_allclose(z, d[f"z:{l}"][h], atol=2e-6, rtol=1e-6)


@pytest.mark.gpu
def test_gpu_model_matches_reference_logits():
    from nanogpt.model import GPT, GPTConfig
    d, sd, cfg, freeze = _load()
    mc = GPTConfig(block_size=cfg["block"], vocab_size=cfg["vocab"], n_layer=cfg["n_layer"],
                   n_head=cfg["n_head"], n_embd=cfg["n_embd"], bias=False,
                   position_encoding="rope", rand_attn_prior_repr="decomposed")
    m = GPT(mc)
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all(k.endswith(("wpe.weight", "dyn_frozen", "dyn_decomp", "dyn_alpha",
                                              "dyn_rho", "dyn_z", "dyn_pattern_slot"))
                                  for k in missing), missing
    m = m.to("cuda", torch.bfloat16).eval()
    for l, blk in enumerate(m.transformer.h):
        a = blk.attn
        for h, (al, rh, zz) in freeze[l]["decomp"].items():
            a.freeze_heads_decomposed([h], al[None].cuda(), rh[None].cuda(), zz[None].cuda())
        for h, p in freeze[l]["patterns"].items():
            a.freeze_heads([h], p[None].cuda())
    x = torch.from_numpy(d["tokens"]).cuda()
    with torch.inference_mode():
        got = m.forward_all_positions(x).double().cpu().flatten()
    for ref in (d["logits_split"], d["logits_eager"]):
        r = torch.from_numpy(ref).double().flatten()
        cos = float(got @ r / (got.norm() * r.norm()))
        assert cos >= 0.9999, f"cosine {cos:.6f}"
