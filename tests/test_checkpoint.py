"""Loader of the reference's nanoGPT checkpoints (nanogpt/checkpoint.py).

The released exports are not available offline, so the checkpoints here are
synthetic files in the reference's layout, built from a model of this repo:
``model_args`` + ``model`` (state dict with the ``_orig_mod.`` compile
prefix), the dense prior as the reference's (n_head, S, S) ``dyn_pattern``
with zero rows for other heads, the derived (n_head, 64, S) ``dyn_rho_band``
(/root/reference/nanogpt/model.py:647-672, :900-911), and the reference's
GPTConfig defaults for absent fields (:1248-1285).

CPU: bit-exact round trip of every weight and freeze buffer, non-dynamic and
learned-absolute exports, refusals.  GPU: logits of a loaded export with
learned (non-closed-form) decomposed heads against the fp32 oracle.
"""
import pickle

import pytest
import torch

from oracle import model_oracle
from test_model import _cos, _oracle_inputs, _small_model


def _reference_layout(m, compile_prefix=True):
    """State dict of model m as the reference's GPT would save it."""
    sd = {}
    for k, v in m.state_dict().items():
        if k.endswith(".attn.dyn_pattern") or k.endswith(".attn.dyn_pattern_slot"):
            continue
        sd[k] = v.clone()
    for i, blk in enumerate(m.transformer.h):
        a = blk.attn
        H, S = a.n_head, a.block_size
        pre = f"transformer.h.{i}.attn."
        if a.dyn_pattern is not None:
            full = torch.zeros(H, S, S, dtype=a.dyn_pattern.dtype)
            for h in range(H):
                s = int(a.dyn_pattern_slot[h])
                if s >= 0:
                    full[h] = a.dyn_pattern[s]
            sd[pre + "dyn_pattern"] = full
        if a.dyn_alpha is not None:
            sd[pre + "dyn_rho_band"] = torch.zeros(H, 64, S)
    if compile_prefix:
        sd = {"_orig_mod." + k: v for k, v in sd.items()}
    return sd


def _model_args(cfg, **over):
    ma = {"block_size": cfg.block_size, "vocab_size": cfg.vocab_size, "n_layer": cfg.n_layer,
          "n_head": cfg.n_head, "n_embd": cfg.n_embd, "dropout": 0.0, "bias": cfg.bias,
          "position_encoding": cfg.position_encoding, "rand_attn_dynamic": True,
          "rand_attn_prior_repr": cfg.rand_attn_prior_repr, "freeze_pattern_dtype": "float32",
          "state_size": 0, "rand_head_rate": 0.0, "rand_mask_rate": 1.0, "rand_components": "none"}
    ma.update(over)
    return ma


def _save(tmp_path, m, name="ckpt.pt", **extra):
    ck = {"model": _reference_layout(m), "model_args": _model_args(m.config), "iter_num": 1000,
          "best_val_loss": 3.1, "config": {"dataset": "openwebtext"}}
    ck.update(extra)
    p = tmp_path / name
    torch.save(ck, p)
    return p


def test_round_trip_is_bit_exact(tmp_path):
    from nanogpt.checkpoint import load_model
    m0, _ = _small_model(T=128, layers=3)
    p = _save(tmp_path, m0)
    m1, cfg, ck = load_model(p, "cpu")
    assert cfg.rand_attn_prior_repr == "decomposed" and cfg.position_encoding == "rope"
    assert ck["iter_num"] == 1000
    s0, s1 = m0.state_dict(), m1.state_dict()
    assert set(s0) == set(s1)
    for k in s0:
        assert s0[k].dtype == s1[k].dtype and torch.equal(s0[k], s1[k]), k
    for b0, b1 in zip(m0.transformer.h, m1.transformer.h):
        b0.attn._refresh_freeze_cache()
        b1.attn._refresh_freeze_cache()
        assert torch.equal(b0.attn._hidx_i32, b1.attn._hidx_i32)
        assert b1.attn._closed[0][:3].tolist() == b0.attn._closed[0][:3].tolist()
    x = torch.randint(0, 50257, (1, 96))
    sd0, ocfg, fz0 = _oracle_inputs(m0)
    sd1, _, fz1 = _oracle_inputs(m1)
    y0 = model_oracle.gpt_forward(sd0, ocfg, fz0, x, path="split", all_positions=False)
    y1 = model_oracle.gpt_forward(sd1, ocfg, fz1, x, path="split", all_positions=False)
    assert torch.equal(y0, y1)


def test_dense_prior_export_and_defaults(tmp_path):
    """A dense-prior export (rand_attn_prior_repr='dense', no decomposed
    buffers) and a non-dynamic learned-absolute export with fields absent
    (reference defaults apply)."""
    from nanogpt.checkpoint import load_model
    from nanogpt.model import GPT, GPTConfig
    torch.manual_seed(0)
    cfg = GPTConfig(block_size=64, vocab_size=500, n_layer=2, n_head=4, n_embd=128, bias=True,
                    rand_attn_prior_repr="dense")
    m0 = GPT(cfg).eval()
    m0.transformer.h[1].attn.freeze_heads([2], torch.rand(1, 64, 64))
    p = _save(tmp_path, m0)
    m1, cfg1, _ = load_model(p, "cpu")
    assert cfg1.rand_attn_prior_repr == "dense"
    a = m1.transformer.h[1].attn
    assert a.dyn_pattern.shape == (1, 64, 64) and a.dyn_pattern_slot.tolist() == [-1, -1, 0, -1]
    assert torch.equal(a.dyn_pattern[0], m0.transformer.h[1].attn.dyn_pattern[0])

    cfg2 = GPTConfig(block_size=64, vocab_size=500, n_layer=1, n_head=4, n_embd=128,
                     position_encoding="learned_absolute")
    m2 = GPT(cfg2).eval()
    sd = {k: v for k, v in m2.state_dict().items() if ".attn.dyn_" not in k}
    ck = {"model": sd, "model_args": {"block_size": 64, "vocab_size": 500, "n_layer": 1, "n_head": 4,
                                      "n_embd": 128}}
    torch.save(ck, tmp_path / "plain.pt")
    m3, cfg3, _ = load_model(tmp_path / "plain.pt", "cpu")
    assert cfg3.position_encoding == "learned_absolute" and cfg3.bias is True
    assert not m3.transformer.h[0].attn.dyn_frozen.any()
    assert torch.equal(m3.transformer.wpe.weight, m2.transformer.wpe.weight)


@pytest.mark.parametrize("field,value", [("rand_head_rate", 0.25), ("state_size", 16),
                                         ("rand_attn_pattern", "uniform"), ("block_type", "mamba"),
                                         ("rand_attn_head_rate_per_layer", "0.25,0.5")])
def test_unsupported_architectures_refused(tmp_path, field, value):
    from nanogpt.checkpoint import load_model
    m0, _ = _small_model(T=64, layers=1)
    ck = {"model": _reference_layout(m0), "model_args": _model_args(m0.config, **{field: value})}
    torch.save(ck, tmp_path / "x.pt")
    with pytest.raises(NotImplementedError, match=field):
        load_model(tmp_path / "x.pt", "cpu")


def test_config_only_fields_and_empty_pattern(tmp_path):
    """Fields persisted only in the full config dict are pulled in
    (eval_nanogpt_logprobs.py:66-70): a per-layer head rate there is refused;
    rand_attn_pattern "" means "none" (model.py:457) and loads."""
    from nanogpt.checkpoint import load_model
    m0, _ = _small_model(T=64, layers=1)
    ck = {"model": _reference_layout(m0), "model_args": _model_args(m0.config),
          "config": {"rand_attn_head_rate_per_layer": "0.1"}}
    torch.save(ck, tmp_path / "h.pt")
    with pytest.raises(NotImplementedError, match="rand_attn_head_rate_per_layer"):
        load_model(tmp_path / "h.pt", "cpu")
    ck = {"model": _reference_layout(m0), "model_args": _model_args(m0.config, rand_attn_pattern=""),
          "config": {"rand_attn_pattern_sharing": "none", "rand_attn_prior_path": ""}}
    torch.save(ck, tmp_path / "e.pt")
    m1, _, _ = load_model(tmp_path / "e.pt", "cpu")
    for k, v in m0.state_dict().items():
        assert torch.equal(m1.state_dict()[k], v), k


def test_packed_layout_and_pickled_objects_refused(tmp_path):
    from nanogpt.checkpoint import load_model
    m0, _ = _small_model(T=64, layers=1)
    p = _save(tmp_path, m0, attention_layout={"mode": "prune", "heads": [[0]]})
    with pytest.raises(NotImplementedError, match="prune"):
        load_model(p, "cpu")
    p = _save(tmp_path, m0, name="obj.pt", extra=torch.nn.Identity())
    with pytest.raises(pickle.UnpicklingError):
        load_model(p, "cpu")


@pytest.mark.gpu
def test_gpu_loaded_export_matches_oracle(tmp_path):
    """A 4-layer export whose decomposed heads carry learned (non-closed-form)
    alpha / rho, loaded onto the GPU in bf16: all-position logits against the
    fp32 oracle, cosine >= 0.9999."""
    from nanogpt.checkpoint import load_model
    m0, x = _small_model(T=256, layers=4)
    g = torch.Generator().manual_seed(9)
    for blk in m0.transformer.h:
        a = blk.attn
        alpha = torch.randn(2, 256, generator=g) * 0.7
        rho = -torch.rand(2, 256, generator=g) * 0.05 * torch.arange(256.0)
        a.freeze_heads_decomposed([10, 11], alpha, rho)
    p = _save(tmp_path, m0)
    m1, _, _ = load_model(p, "cuda", dtype=torch.bfloat16)
    assert m1.transformer.h[0].attn.dyn_z.dtype == torch.float32
    with torch.inference_mode():
        got = m1.forward_all_positions(x.cuda()).float().cpu()
    sd, ocfg, freeze = _oracle_inputs(m0)
    ref = model_oracle.gpt_forward(sd, ocfg, freeze, x, path="eager", all_positions=True)
    assert _cos(got, ref) >= 0.9999


def test_reference_writer_matches_layout_and_round_trips(tmp_path):
    """save_reference_checkpoint writes the layout of _reference_layout (the
    test's own statement of the reference export) and load_model restores
    every weight and freeze buffer bit for bit."""
    from nanogpt.checkpoint import load_model, reference_state_dict, save_reference_checkpoint
    m0, _ = _small_model(T=64, layers=2)
    want = _reference_layout(m0)
    got = reference_state_dict(m0, compile_prefix=True)
    assert set(got) == set(want)
    for k, v in want.items():
        if k.endswith("dyn_rho_band"):
            assert got[k].shape == v.shape
            continue
        assert torch.equal(got[k], v), k
    p = save_reference_checkpoint(m0, tmp_path / "w.pt", iter_num=7)
    m1, cfg1, ck = load_model(p, "cpu")
    assert ck["iter_num"] == 7
    for k, v in m0.state_dict().items():
        assert torch.equal(m1.state_dict()[k], v), k
