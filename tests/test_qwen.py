"""CPU checks of the Qwen3 GQA caller (selective-attention-freezing_amd/qwen) and
its oracle.

Pinned by tests/golden/qwen_forward_small.npz, written by the reference's own
hybrid adapter (qwen/nanogpt/hybrid_prior_attention.py) on CPU:
  * the oracle restatement reproduces the reference's last hidden states for
    the unconverted model, dense priors and decomposed priors;
  * this build's adapter reproduces the reference's routing tables (frozen /
    hidx / pidx / kvidx, bit-exact), its dense prior normalisation (bit-exact)
    and, on its torch split path, the reference's hidden states;
  * the frozen-set schedule follows bench_qwen_prefill_triton.py:143-159.
"""
import numpy as np
import pytest
import torch

import qwen_cases as qc
from oracle import qwen_oracle as qo


@pytest.fixture(scope="module")
def golden():
    return qc.load_golden()


@pytest.mark.parametrize("repr", ["base", "dense", "decomp"])
def test_oracle_matches_reference_golden(golden, repr):
    _, ocfg = qc.golden_cfg(golden)
    sd = qc.golden_state_dict(golden)
    ids = torch.from_numpy(golden["tokens"])
    fr = None if repr == "base" else qc.golden_freeze(golden, repr)[1]
    y = qo.qwen_forward(sd, ocfg, fr, ids)
    ref = torch.from_numpy(golden[f"hidden_{repr}"])
    assert (y - ref).abs().max().item() < 2e-5


def test_oracle_fails_a_planted_gqa_mistake(golden):
    # frozen heads reading the wrong KV group must not pass the golden check
    _, ocfg = qc.golden_cfg(golden)
    sd = qc.golden_state_dict(golden)
    ids = torch.from_numpy(golden["tokens"])
    fr = qc.golden_freeze(golden, "dense")[1]
    for l in range(ocfg["n_layers"]):
        p = f"model.layers.{l}.self_attn.v_proj.weight"
        sd[p] = sd[p].view(2, -1, sd[p].size(-1)).flip(0).reshape(sd[p].shape)
    y = qo.qwen_forward(sd, ocfg, fr, ids)
    assert (y - torch.from_numpy(golden["hidden_dense"])).abs().max().item() > 1e-2


@pytest.mark.parametrize("repr", ["dense", "decomp"])
def test_adapter_tables_and_split_path_match_reference(golden, repr):
    import qwen
    m = qc.golden_model(golden)
    saved, _ = qc.convert_golden(m, golden, repr, "cpu", torch.float32)
    for l, blk in enumerate(m.model.layers):
        a = blk.self_attn
        assert type(a).__name__ == "HybridQwen3Attention"
        for name in ("frozen", "hidx", "pidx", "kvidx"):
            got = getattr(a, f"{name}_mask_i32" if name == "frozen" else f"{name}_i32").numpy()
            assert np.array_equal(got, golden[f"{repr}:{name}:{l}"]), (l, name)
        if repr == "dense":
            assert np.array_equal(a.prior_pattern.numpy(), golden[f"dense:prior:{l}"])
        else:
            assert np.allclose(a.dec_z.numpy(), golden[f"decomp:z:{l}"], atol=1e-5, rtol=0)
    with torch.inference_mode():
        y = qwen.backbone_forward(m.model, torch.from_numpy(golden["tokens"]))
    assert (y - torch.from_numpy(golden[f"hidden_{repr}"])).abs().max().item() < 2e-5
    qwen.restore_originals(saved)
    with torch.inference_mode():
        y0 = qwen.backbone_forward(m.model, torch.from_numpy(golden["tokens"]))
    assert (y0 - torch.from_numpy(golden["hidden_base"])).abs().max().item() < 2e-5


def test_closed_form_classification_of_mean_priors():
    import qwen
    cfg = qwen.qwen_config(n_layers=2, hidden=64, n_heads=4, n_kv_heads=2, head_dim=32,
                           intermediate=96, vocab=128)
    m = qwen.build_model(cfg, device="cpu", dtype=torch.float32)
    saved, masks = qwen.convert_with_rate(m, 0.5, 32, repr="decomposed")
    for blk, mask in zip(m.model.layers, masks):
        kind, param = blk.self_attn._closed
        assert np.array_equal(kind, np.where(mask.numpy(), 1, 0))
        assert np.array_equal(blk.self_attn.frozen_mask_i32.numpy(), 2 * mask.numpy().astype(np.int32))
    ids = torch.randint(0, 128, (2, 32))
    with torch.inference_mode():
        yd = qwen.backbone_forward(m.model, ids)
    qwen.restore_originals(saved)
    saved, _ = qwen.convert_with_rate(m, 0.5, 32, repr="dense")
    with torch.inference_mode():
        yp = qwen.backbone_forward(m.model, ids)
    assert (yd - yp).abs().max().item() < 1e-5


def test_nested_head_masks_schedule():
    import qwen
    H, L = 14, 24
    assert [qwen.n_frozen_for(r, H) for r in (0.0, 0.25, 0.5, 0.75)] == [0, 4, 7, 10]
    prev = None
    for r in (0.25, 0.5, 0.75):
        ms = qwen.nested_head_masks(r, L, H, seed=1337)
        assert all(int(m.sum()) == qwen.n_frozen_for(r, H) for m in ms)
        if prev is not None:
            assert all(bool((p <= m).all()) for p, m in zip(prev, ms))   # nested
        prev = ms
    g = torch.Generator().manual_seed(1337 + 104729 * 3)
    order = torch.randperm(H, generator=g)
    assert set(torch.nonzero(prev[3]).flatten().tolist()) == set(order[:10].tolist())


def test_hip_prologue_refuses_cpu_tensors():
    import kernel
    q = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    cs = torch.zeros(8, 64)
    with pytest.raises(RuntimeError, match="HIP devices only"):
        kernel.qk_rmsnorm_rope_(q, q, w, w, 1e-6, cs, cs)
