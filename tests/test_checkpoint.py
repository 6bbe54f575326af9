"""Loader of the reference's nanoGPT checkpoints (nanogpt/checkpoint.py).

The released exports are not available offline.  The loader is pinned on
tests/golden/gpt_export_small.npz, which the reference's own GPT wrote
(tests/golden/make_golden.py): its state dicts under their own key names
(``transformer.h.{i}.main_block.*``, every buffer the reference saves:
dyn_frozen, dyn_decomp / dyn_alpha / dyn_rho / dyn_z, the lazily created
dyn_rho_band and dyn_pattern, the dense representation's (n_head, S, S)
dyn_pattern), its GPTConfig as model_args and its split-path logits.  A
checkpoint file is assembled from them as nanogpt/train.py saves one
(``model`` with torch.compile's ``_orig_mod.`` prefix, ``model_args``,
optimizer state, ``config``, RNG state) and read back with
``weights_only=True``.

CPU: the loaded model reproduces the reference's logits through the oracle;
reference_state_dict writes back exactly the reference's keys and values;
synthetic exports (written by the now-pinned reference_state_dict) round-trip
bit for bit; refusals.  GPU: the bf16 HIP model of a loaded export against the
reference's logits, and an export with learned alpha / rho heads against the
fp32 oracle.
"""
import json
import os
import pickle

import numpy as np
import pytest
import torch

from oracle import model_oracle
from test_model import _cos, _oracle_inputs, _small_model

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gpt_export_small.npz")


def _fixture(tag):
    """(reference state dict, model_args, tokens, logits_split) of one model
    of the export fixture; every floating tensor of the reference model is
    fp32 (float16-stored entries are exact)."""
    d = np.load(FIX, allow_pickle=False)
    f16 = set(json.loads(str(d[f"{tag}/f16keys"])))
    pre = f"{tag}/sd/"
    sd = {}
    for k in d.files:
        if k.startswith(pre):
            name = k[len(pre):]
            t = torch.from_numpy(d[k].copy())
            sd[name] = t.float() if name in f16 else t
    return (sd, json.loads(str(d[f"{tag}/model_args"])), torch.from_numpy(d[f"{tag}/tokens"]),
            torch.from_numpy(d[f"{tag}/logits_split"]))


def _train_py_checkpoint(path, sd, model_args):
    """A checkpoint file laid out as nanogpt/train.py:688-700 writes it."""
    ck = {"model": {"_orig_mod." + k: v for k, v in sd.items()},
          "optimizer": {"state": {0: {"step": torch.tensor(5.0), "exp_avg": torch.zeros(3)}},
                        "param_groups": [{"lr": 6e-4, "params": [0]}]},
          "model_args": model_args, "attention_layout": None, "iter_num": 5000, "best_val_loss": 3.02,
          "config": {"dataset": "openwebtext", "batch_size": 12},
          "cpu_rng_state": torch.random.get_rng_state(), "cuda_rng_states": None}
    torch.save(ck, path)
    return path


@pytest.mark.parametrize("tag", ["decomposed", "dense"])
def test_reference_export_loads_and_reproduces_logits(tmp_path, tag):
    """The reference's own export loads strictly and the loaded weights and
    freeze state give the reference's split-path logits (oracle, fp32)."""
    from nanogpt.checkpoint import load_model
    sd, ma, x, want = _fixture(tag)
    assert any(".main_block." in k for k in sd) and not any(".attn." in k for k in sd)
    m, cfg, ck = load_model(_train_py_checkpoint(tmp_path / "ref.pt", sd, ma), "cpu")
    assert cfg.rand_attn_prior_repr == tag and ck["iter_num"] == 5000
    got_sd, ocfg, freeze = _oracle_inputs(m)
    for k, v in sd.items():
        mine = k.replace(".main_block.", ".attn.")
        if mine in got_sd and not k.endswith("dyn_pattern"):
            assert torch.equal(got_sd[mine], v.float()), k
    got = model_oracle.gpt_forward(got_sd, ocfg, freeze, x, path="split", all_positions=True)
    np.testing.assert_allclose(got.numpy(), want.numpy(), atol=2e-5, rtol=1e-5)


@pytest.mark.parametrize("tag", ["decomposed", "dense"])
def test_reference_state_dict_is_the_reference_layout(tag):
    """Written back, a loaded export has exactly the reference's key set,
    dtypes and values (dense patterns expanded to (n_head, S, S), the rho
    band rebuilt from rho)."""
    from nanogpt.checkpoint import convert_state_dict, reference_state_dict, build_config_from_ckpt
    from nanogpt.model import GPT
    sd, ma, _, _ = _fixture(tag)
    m = GPT(build_config_from_ckpt({"model_args": ma}))
    m.load_state_dict(convert_state_dict(sd, m), strict=True)
    got = reference_state_dict(m)
    assert set(got) == set(sd), (set(got) ^ set(sd))
    for k, v in sd.items():
        assert got[k].dtype == v.dtype and got[k].shape == v.shape, k
        assert torch.equal(got[k], v), k
    pref = reference_state_dict(m, compile_prefix=True)
    assert set(pref) == {"_orig_mod." + k for k in sd}


def _save(tmp_path, m, name="ckpt.pt", **extra):
    from nanogpt.checkpoint import reference_state_dict
    ck = {"model": reference_state_dict(m, compile_prefix=True), "model_args": _model_args(m.config),
          "iter_num": 1000, "best_val_loss": 3.1, "config": {"dataset": "openwebtext"}}
    ck.update(extra)
    p = tmp_path / name
    torch.save(ck, p)
    return p


def _model_args(cfg, **over):
    ma = {"block_size": cfg.block_size, "vocab_size": cfg.vocab_size, "n_layer": cfg.n_layer,
          "n_head": cfg.n_head, "n_embd": cfg.n_embd, "dropout": 0.0, "bias": cfg.bias,
          "position_encoding": cfg.position_encoding, "rand_attn_dynamic": True,
          "rand_attn_prior_repr": cfg.rand_attn_prior_repr, "freeze_pattern_dtype": "float32",
          "state_size": 0, "rand_head_rate": 0.0, "rand_mask_rate": 1.0, "rand_components": "none"}
    ma.update(over)
    return ma


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
    from nanogpt.checkpoint import load_model, reference_state_dict
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
    # a non-dynamic reference model saves no dyn_* buffer at all
    sd = {k: v for k, v in reference_state_dict(m2).items() if ".main_block.dyn_" not in k}
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
    from nanogpt.checkpoint import load_model, reference_state_dict
    m0, _ = _small_model(T=64, layers=1)
    ck = {"model": reference_state_dict(m0, compile_prefix=True),
          "model_args": _model_args(m0.config, **{field: value})}
    torch.save(ck, tmp_path / "x.pt")
    with pytest.raises(NotImplementedError, match=field):
        load_model(tmp_path / "x.pt", "cpu")


def test_config_only_fields_and_empty_pattern(tmp_path):
    """Fields persisted only in the full config dict are pulled in
    (eval_nanogpt_logprobs.py:66-70): a per-layer head rate there is refused;
    rand_attn_pattern "" means "none" (model.py:457) and loads."""
    from nanogpt.checkpoint import load_model, reference_state_dict
    m0, _ = _small_model(T=64, layers=1)
    ck = {"model": reference_state_dict(m0, compile_prefix=True), "model_args": _model_args(m0.config),
          "config": {"rand_attn_head_rate_per_layer": "0.1"}}
    torch.save(ck, tmp_path / "h.pt")
    with pytest.raises(NotImplementedError, match="rand_attn_head_rate_per_layer"):
        load_model(tmp_path / "h.pt", "cpu")
    ck = {"model": reference_state_dict(m0, compile_prefix=True),
          "model_args": _model_args(m0.config, rand_attn_pattern=""),
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


def test_reference_writer_round_trips(tmp_path):
    """save_reference_checkpoint (reference_state_dict, pinned above on the
    reference's own export) writes a file load_model restores bit for bit."""
    from nanogpt.checkpoint import load_model, save_reference_checkpoint
    m0, _ = _small_model(T=64, layers=2)
    p = save_reference_checkpoint(m0, tmp_path / "w.pt", iter_num=7)
    ck = torch.load(p, weights_only=True)
    assert all(k.startswith("_orig_mod.") for k in ck["model"])
    assert not any(".attn." in k for k in ck["model"])
    m1, cfg1, ck = load_model(p, "cpu")
    assert ck["iter_num"] == 7
    for k, v in m0.state_dict().items():
        assert torch.equal(m1.state_dict()[k], v), k


def test_loaded_dense_patterns_keep_padded_rows(tmp_path):
    """Dense patterns of a loaded export sit in the padded slots freeze_heads
    allocates (rows at a 4 KB-multiple pitch get 256 bytes more), and a later
    dtype cast keeps that layout."""
    from nanogpt.checkpoint import load_model
    from nanogpt.model import GPT, GPTConfig
    torch.manual_seed(1)
    cfg = GPTConfig(block_size=1024, vocab_size=64, n_layer=1, n_head=2, n_embd=64, bias=False,
                    rand_attn_prior_repr="decomposed")
    m0 = GPT(cfg).eval()
    pat = torch.rand(1, 1024, 1024)
    m0.transformer.h[0].attn.freeze_heads([1], pat)
    m1, _, _ = load_model(_save(tmp_path, m0), "cpu")
    a = m1.transformer.h[0].attn
    assert a.dyn_pattern.shape == (1, 1024, 1024) and a.dyn_pattern.stride() == (1024 * 1088, 1088, 1)
    assert torch.equal(a.dyn_pattern, m0.transformer.h[0].attn.dyn_pattern)
    m1.to(dtype=torch.float64)   # 8 KB rows: padded again (a cast returns contiguous tensors)
    assert a.dyn_pattern.dtype == torch.float64 and a.dyn_pattern.stride(1) == 1024 + 32
    assert torch.equal(a.dyn_pattern, m0.transformer.h[0].attn.dyn_pattern.double())
    m1.to(dtype=torch.bfloat16)  # 2 KB rows: no padding
    assert a.dyn_pattern.dtype == torch.bfloat16 and a.dyn_pattern.stride(1) == 1024


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["decomposed", "dense"])
def test_gpu_reference_export_matches_reference_logits(tmp_path, tag):
    """The reference's own export, loaded onto the GPU in bf16 and run through
    the HIP path: all-position logits against the reference's fp32 split-path
    logits, cosine >= 0.9999."""
    from nanogpt.checkpoint import load_model
    sd, ma, x, want = _fixture(tag)
    m, _, _ = load_model(_train_py_checkpoint(tmp_path / "ref.pt", sd, ma), "cuda", dtype=torch.bfloat16)
    with torch.inference_mode():
        got = m.forward_all_positions(x.cuda()).float().cpu()
    c = _cos(got, want)
    assert c >= 0.9999, f"logits cosine {c:.6f}"
