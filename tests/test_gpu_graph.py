"""HIP graph capture of the prefill (the reference's checkpoint bench
captures one, nanogpt/bench_checkpoint_prefill.py:87-109).

A model with live, dense, generic decomposed and closed-form heads (the
closed-form scan runs on a second stream joined inside the capture) is
captured once; the graph is replayed three times with eager prefills and
synchronisations in between, and every replay is compared with the eager
output of the same tokens (the scan's look-back order can move a last bit:
cosine >= 0.99999) and with the fp32 oracle."""
import pytest
import torch

from oracle import model_oracle
from test_model import _cos, _oracle_inputs, _small_model

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager():
    m, x = _small_model(T=256, layers=3, device="cuda", dtype=torch.bfloat16)
    x2 = torch.randint(0, 50257, x.shape, generator=torch.Generator().manual_seed(11)).cuda()
    with torch.inference_mode():
        eager = m.forward_all_positions(x).float().cpu()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                m.forward_all_positions(x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = m.forward_all_positions(x)
        torch.cuda.synchronize()
        for rep in range(3):
            other = m.forward_all_positions(x2)      # eager work between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = out.float().cpu()
            assert _cos(got, eager) >= 0.99999, f"replay {rep}"
            assert torch.isfinite(other).all()
    sd, ocfg, freeze = _oracle_inputs(m)
    ref = model_oracle.gpt_forward(sd, ocfg, freeze, x.cpu(), path="eager", all_positions=True)
    assert _cos(got, ref) >= 0.9999
