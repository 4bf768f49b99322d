"""The LTX-2 video block captured in a HIP graph (``torch.cuda.graph``): every replay gives the
eager block's output bit for bit, with eager blocks and synchronizations between the replays, and
a replay after new values are copied into the captured input buffer gives the eager output for
those values. The block's launches take torch's current stream, so capture records them as they
are; quantized layers dequantize into the capture stream's own workspace."""

import pytest
import torch

from kinomlx_amd import workloads
from kinomlx_amd.ltx2.transformer import TransformerArgs
from tests._blocks import device_tables, ltx_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(
    "spec",
    [
        workloads.LTXSpec(grid=(2, 4, 16), text_tokens=32, dim=4096, heads=32, head_dim=128),
        workloads.LTXSpec(grid=(2, 4, 16), text_tokens=32, dim=4096, heads=32, head_dim=128, bits=4),
    ],
    ids=["d4096", "d4096-int4"],
)
def test_ltx_block_graph_replays_match_eager(device, spec):
    p, _, inputs, pe = ltx_case(spec)
    block = workloads.build_ltx_block(spec, p, device)
    x = inputs["x"].to(device)
    args = TransformerArgs(x=x, context=inputs["context"].to(device), timesteps=p["timesteps"].to(device),
                           positional_embeddings=device_tables(pe, device))

    def step():
        return block(args)[0].x

    eager = step().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    torch.cuda.synchronize()
    for replay in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {replay}"
        again = step()
        torch.cuda.synchronize()
        assert torch.equal(again, eager), f"eager block after replay {replay}"

    x.copy_(torch.flip(x, dims=[1]) * 0.5)
    fresh = step().clone()
    assert not torch.equal(fresh, eager)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(captured, fresh)
    del graph
