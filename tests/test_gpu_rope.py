"""GPU parity of the in-place RoPE kernel (saf_rope_qk_inplace) against the
oracle's Llama half rotation (nanogpt/model.py:57-99), on the interleaved
q/k views of one projection output that the model passes and on contiguous
tensors, for every supported head dim and fp32 / bf16 caches."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc
from saf_cases import compare, f64

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hd", [32, 64, 96, 128])
@pytest.mark.parametrize("cache", ["f32", "bf16"])
@pytest.mark.parametrize("layout", ["interleaved", "contiguous"])
def test_rope_matches_oracle(hd, cache, layout):
    import kernel
    B, U, T = 2, 5, 333
    g = torch.Generator().manual_seed(hd + T)
    q = torch.randn(B, U, T, hd, generator=g).bfloat16()
    k = torch.randn(B, U, T, hd, generator=g).bfloat16()
    cos, sin = orc.rope_cache(hd, T + 7)
    ct = torch.from_numpy(cos).float()
    st = torch.from_numpy(sin).float()
    if cache == "bf16":
        ct, st = ct.bfloat16(), st.bfloat16()
    if layout == "interleaved":
        buf = torch.stack([q, k], dim=2).permute(0, 3, 2, 1, 4).contiguous().cuda()  # (B, T, 2, U, hd)
        qd, kd = buf[:, :, 0].transpose(1, 2), buf[:, :, 1].transpose(1, 2)
    else:
        qd, kd = q.cuda(), k.cuda()
    kernel.rope_qk_(qd, kd, ct.cuda().view(1, 1, T + 7, hd), st.cuda().view(1, 1, T + 7, hd))
    torch.cuda.synchronize()
    c, s = f64(ct)[:T], f64(st)[:T]
    compare(qd, orc.apply_rope(f64(q), c, s), what=f"rope q hd{hd}")
    compare(kd, orc.apply_rope(f64(k), c, s), what=f"rope k hd{hd}")


def test_rope_rejects_bad_cache():
    import kernel
    q = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="cos/sin"):
        kernel.rope_qk_(q, q.clone(), torch.zeros(4, 64, device="cuda"), torch.zeros(4, 64, device="cuda"))
