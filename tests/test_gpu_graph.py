"""The layer step (router projection, route, expert forward) captured into a HIP graph and replayed:
every replay equals the eager step bit for bit, with eager work and synchronisations between the
replays (the library records no memset nodes; its workspaces come from the capture's memory pool)."""
import pytest
import torch

import bench

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["small_bf16", "dsv3_decode_mxfp8"])
def test_layer_step_graph_replays_equal_eager(gpu, name):
    print(f"[graph] {name}", flush=True)
    layer = bench.Layer(name, gpu)
    layer.step()
    torch.cuda.synchronize()
    eager = layer.out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer.step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer.step()
    for i in range(3):
        layer.out.fill_(float(i + 1))  # eager work between replays; the replay must overwrite it
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(layer.out, eager), f"replay {i}"
        layer.step()  # an eager step between replays leaves the graph's result unchanged
        torch.cuda.synchronize()
        assert torch.equal(layer.out, eager)
