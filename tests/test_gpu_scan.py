"""GPU parity of the closed-form scan (frozen mean / decay / window heads) at
long T against the oracle's direct recurrences (oracle.saf_oracle.mean_apply,
decay_apply, window_apply; float64 on the same rounded V).

Covers what the short cases of test_gpu_mixed_attn cannot: many chunks per
sequence with few sequences (deep look-back chains: 64 chunks of one
sequence in flight together), the sizing run's full shape (B=8, H=12,
T=16384), windows longer than a chunk, T not a multiple of the chunk, and V
as a strided view of a fused projection.  Bound: max-abs <= 2e-2 and
relative-L2 <= 1e-2 (bf16 / fp16 output)."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc
from saf_cases import closed_params, compare

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _kernel():
    import kernel
    return kernel


def _heads(H, T, seed):
    """Seeded per-head closed forms as decomposed buffers (alpha, rho, z) of
    length T, classified as the caller's path does: returns the buffers, the
    closed_form tables and the oracle's (kind, param) per head."""
    K = _kernel()
    rng = np.random.default_rng(seed)
    kinds = {}
    for h in range(H):
        k = h % 3 if H <= 3 else int(rng.integers(0, 3))
        if k == 0:
            kinds[h] = ("mean", 0)
        elif k == 1:
            kinds[h] = ("decay", float(rng.uniform(0.001, 0.1)))
        else:
            kinds[h] = ("window", int(rng.integers(64, 1025)))
    alpha, rho, z = closed_params(H, T, kinds)
    cf = K.classify_closed_form(alpha, rho, z)
    names = {K.CLOSED_MEAN: "mean", K.CLOSED_DECAY: "decay", K.CLOSED_WINDOW: "window"}
    spec = []
    for h in range(H):
        kind = names[int(cf[0][h])]
        assert kind == kinds[h][0], f"head {h}: {kinds[h]} classified as {kind}"
        prm = float(cf[1][h])
        spec.append((kind, int(prm) if kind == "window" else prm))
    return (alpha, rho, z), cf, spec


def _oracle(v, spec):
    v64 = v.float().cpu().numpy().astype(np.float64)
    out = np.empty_like(v64)
    for h, (kind, prm) in enumerate(spec):
        x = v64[:, h]
        if kind == "mean":
            out[:, h] = orc.mean_apply(x)
        elif kind == "decay":
            out[:, h] = orc.decay_apply(x, prm)
        else:
            out[:, h] = orc.window_apply(x, prm)
    return out


def _run(B, H, T, hd, dtype, strided, seed):
    K = _kernel()
    g = torch.Generator().manual_seed(seed)
    (alpha, rho, z), cf, spec = _heads(H, T, seed)
    if strided:
        # v as the third slice of a (B, T, 3, H, hd) projection output
        qkv = torch.randn(B, T, 3, H, hd, generator=g).to(dtype)
        v = qkv.to(DEV)[:, :, 2].transpose(1, 2)
        v_cpu = qkv[:, :, 2].transpose(1, 2)
    else:
        v_cpu = torch.randn(B, H, T, hd, generator=g).to(dtype)
        v = v_cpu.to(DEV)
    frozen = torch.full((H,), 2, dtype=torch.int32, device=DEV)
    qk = torch.empty(B, 0, T, hd, dtype=dtype, device=DEV)  # no live heads: empty compact q / k
    y = K.fused_mixed_attn(qk, qk, v, None, frozen, alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV),
                           closed_form=cf)
    torch.cuda.synchronize()
    compare(y, _oracle(v_cpu, spec), what=f"B{B} H{H} T{T} hd{hd} {dtype} strided={strided} {spec}")


@pytest.mark.parametrize("B,H,T,hd,strided", [
    (1, 3, 16384, 64, False),    # 64 chunks of 3 sequences: deep look-back
    (1, 4, 16000, 128, True),    # T not a multiple of the chunk, strided V
    (2, 3, 12345, 32, False),
    (1, 2, 9000, 96, True),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_scan_long_sequences(B, H, T, hd, strided, dtype):
    _run(B, H, T, hd, dtype, strided, seed=T + hd + B)


def test_scan_sizing_run_shape():
    """The frozen-only sizing run's shape (B=8, H=12, T=16384, hd=64)."""
    _run(8, 12, 16384, 64, torch.bfloat16, False, seed=1337)


def test_scan_repeat_calls_agree():
    """Back-to-back calls reuse the workspace: the clear before each scan
    leaves no stale status word, so repeated calls give the same output up
    to the look-back's last-bit rounding order."""
    K = _kernel()
    B, H, T, hd = 2, 6, 8192, 64
    (alpha, rho, z), cf, spec = _heads(H, T, 7)
    v = torch.randn(B, H, T, hd, generator=torch.Generator().manual_seed(7)).bfloat16().to(DEV)
    frozen = torch.full((H,), 2, dtype=torch.int32, device=DEV)
    qk = torch.empty(B, 0, T, hd, dtype=v.dtype, device=DEV)
    bufs = dict(alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV))
    ys = [K.fused_mixed_attn(qk, qk, v, None, frozen, closed_form=cf, **bufs) for _ in range(3)]
    torch.cuda.synchronize()
    ref = _oracle(v.cpu(), spec)
    for y in ys:
        compare(y, ref, what="repeat call")
    for y in ys[1:]:
        assert (y.float() - ys[0].float()).abs().max().item() <= 2e-2


def test_scan_give_up_is_loud():
    """A look-back wait that gives up must never return a silently incomplete
    sum.  The host-set drill (scan_spin_limit < 0) makes every chunk after the
    first give up at once; every kernel still exits normally (the stream
    synchronises), the call raises under validate=True, the rows of the
    first chunk are still right and every later row is NaN.  A normal call
    on the next workspace is exact again."""
    K = _kernel()
    B, H, T, hd = 2, 3, 4096, 64
    (alpha, rho, z), cf, spec = _heads(H, T, 11)
    v_cpu = torch.randn(B, H, T, hd, generator=torch.Generator().manual_seed(11)).bfloat16()
    v = v_cpu.to(DEV)
    frozen = torch.full((H,), 2, dtype=torch.int32, device=DEV)
    qk = torch.empty(B, 0, T, hd, dtype=v.dtype, device=DEV)
    bufs = dict(alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV), closed_form=cf)
    with pytest.raises(RuntimeError, match="gave up"):
        K.fused_mixed_attn(qk, qk, v, None, frozen, scan_spin_limit=-1, **bufs)
    torch.cuda.synchronize()
    y = K.fused_mixed_attn(qk, qk, v, None, frozen, scan_spin_limit=-1, validate=False, **bufs)
    torch.cuda.synchronize()
    ref = _oracle(v_cpu, spec)
    ch = 256   # scan rows per chunk at hd 64
    compare(y[:, :, :ch], ref[:, :, :ch], what="first chunk under the give-up drill")
    assert torch.isnan(y[:, :, ch:].float()).all()
    y2 = K.fused_mixed_attn(qk, qk, v, None, frozen, **bufs)
    torch.cuda.synchronize()
    compare(y2, ref, what="normal call after the drill")
