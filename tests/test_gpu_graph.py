"""The MoE decode layer captured in a HIP graph: every replay (with eager work and synchronisation
between replays) matches the eager result bit for bit (the layer records no memset nodes; the
arrival counters are reset by the kernels themselves)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_moe_layer_graph_replays_match_eager():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helios_glm53flash_amd import moe
    E, hidden, inter, topk = 32, 512, 256, 4
    ex = moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=9)
    sh = moe.synthetic_dense_mlp(hidden, inter, 2, seed=10)
    layer = moe.MoeLayer(ex, sh, topk=topk)
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    x = torch.randn((1, hidden), generator=g, device="cuda").half()
    scores = torch.randn((3, 1, E), generator=g, device="cuda").half()
    ws = torch.zeros(layer.workspace_bytes(1), dtype=torch.uint8, device="cuda")
    eager = [layer(x, scores[i], ws=ws).clone() for i in range(3)]
    torch.cuda.synchronize()
    outs = [torch.empty((1, hidden), dtype=torch.float16, device="cuda") for _ in range(3)]
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(3):
            layer(x, scores[i], y=outs[i], ws=ws)
    for rep in range(4):
        for o in outs:
            o.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        for i in range(3):
            assert torch.equal(outs[i], eager[i]), f"replay {rep} step {i}"
        # eager work between replays
        again = layer(x, scores[rep % 3], ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(again, eager[rep % 3])


def test_moe_check_status_reports_and_clears():
    """hx_moe_check_status: 0 after normal few-token layer calls; a set wait-status word (forced from
    the host, no kernel involved) is reported as HX_ERR_TIMEOUT once and cleared."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helios_glm53flash_amd import moe
    from helios_glm53flash_amd._lib import HX_ERR_TIMEOUT, HxError
    E, hidden, inter = 16, 256, 128
    layer = moe.MoeLayer(moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=3),
                         moe.synthetic_dense_mlp(hidden, inter, 2, seed=4), topk=4)
    ws = torch.zeros(layer.workspace_bytes(1), dtype=torch.uint8, device="cuda")
    x = torch.randn((1, hidden), device="cuda").half()
    s = torch.randn((1, E), device="cuda").half()
    layer(x, s, ws=ws)
    moe.check_status(ws)
    ws.view(torch.int32)[10242] = 1  # the status word in the counter area
    with pytest.raises(HxError, match=str(HX_ERR_TIMEOUT)):
        moe.check_status(ws)
    moe.check_status(ws)  # cleared
    assert int(ws.view(torch.int32)[:16384].abs().sum()) == 0  # counter area left zero
