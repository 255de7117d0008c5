"""launch_route_plan_noalloc: the route plan with the pack's own per-device
scratch array instead of a caller workspace.  Its outputs must equal
launch_route_plan's bit for bit (integer and index work), including on
consecutive calls where the second is smaller (the array keeps the last
call's contents), at the documented maximum plan size, and when captured in
a HIP graph and replayed (the use it exists for).  Host-side rejections
(a workspace passed in, a plan above the scratch limit) enqueue nothing."""
import numpy as np
import pytest

import oracle
from pih_amd import abi, synth
from tests.helpers import to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    import torch

    from pih_amd.device import engine_stream

    with engine_stream() as s:
        yield s
        torch.cuda.synchronize()


def _outputs(tokens, topk, experts):
    import torch

    fill = lambda n, dt: torch.full((n,), -1, dtype=dt, device="cuda")
    return (fill(experts + 1, torch.int32), fill(tokens * topk, torch.int32), fill(tokens * topk, torch.float32),
            fill(tokens * topk, torch.int32), torch.zeros(1, dtype=torch.int32, device="cuda"))


def _request(ids_d, wts_d, outs, tokens, topk, experts, ws=None, stream=None):
    from pih_amd.device import ptr, stream_handle

    off, rt, rw, tr, flag = outs
    return abi.request(abi.LN["route_plan"], topk_ids_u32=ptr(ids_d), topk_weights_f32=ptr(wts_d),
                       expert_offsets_u32=ptr(off), row_token_u32=ptr(rt), row_weight_f32=ptr(rw),
                       token_rows_u32=ptr(tr), workspace=ptr(ws), workspace_bytes=0 if ws is None else ws.numel(),
                       error_flag_u32=ptr(flag), stream=stream_handle() if stream is None else stream,
                       token_count=tokens, top_k=topk, expert_count=experts)


def _host(outs):
    import torch

    torch.cuda.synchronize()
    return [to_host(t).copy() for t in outs]


def _plan(noalloc, ids, wts, experts):
    import torch

    from pih_amd.linear import route_plan_workspace

    tokens, topk = ids.shape
    ids_d, wts_d = to_dev(ids), to_dev(wts)
    outs = _outputs(tokens, topk, experts)
    L = abi.linear_pack()
    if noalloc:
        st = L.call("launch_route_plan_noalloc", _request(ids_d, wts_d, outs, tokens, topk, experts))
    else:
        ws = torch.empty(route_plan_workspace(tokens, topk, experts), dtype=torch.uint8, device="cuda")
        st = L.call("launch_route_plan", _request(ids_d, wts_d, outs, tokens, topk, experts, ws))
    assert st.code == abi.OK, st
    return _host(outs)


def _same(a, b):
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("first,second", [((4096, 256, 8), (300, 64, 6)), ((16384, 256, 8), (65, 16, 4))])
def test_noalloc_equals_workspace_entry_twice(eng, first, second):
    """Two calls in a row, the second smaller; the first of the second pair
    is the largest plan the scratch holds (16384 tokens, 256 experts)."""
    for j, (tokens, experts, topk) in enumerate((first, second)):
        ids, wts = synth.zipf_router(synth.config_seed(4, 13000 + 7 * j + tokens), tokens, experts, topk)
        got = _plan(True, ids, wts, experts)
        want = _plan(False, ids, wts, experts)
        _same(got, want)
        assert got[4][0] == 0
        o_ref, rt_ref, rw_ref, tr_ref = oracle.route_plan(ids, wts, experts)
        np.testing.assert_array_equal(got[0].view(np.uint32), o_ref)
        np.testing.assert_array_equal(got[1].view(np.uint32), rt_ref)
        np.testing.assert_array_equal(got[3].view(np.uint32).reshape(tokens, topk), tr_ref)


def test_noalloc_flags_bad_routes_like_workspace_entry(eng):
    ids = np.array([[0, 1], [2, 2], [9, 0], [3, 1]], np.uint32)
    wts = np.array([[0.5, 0.5], [0.5, 0.5], [0.5, 0.5], [np.nan, 0.5]], np.float32)
    got = _plan(True, ids, wts, 8)
    _same(got, _plan(False, ids, wts, 8))
    assert got[4][0] == 7


def test_noalloc_rejects_workspace_and_oversized_plans(eng):
    import torch

    L = abi.linear_pack()
    ids_d = torch.zeros(8, dtype=torch.int32, device="cuda")
    wts_d = torch.zeros(8, dtype=torch.float32, device="cuda")
    outs = _outputs(4, 2, 8)
    ws = torch.empty(1 << 16, dtype=torch.uint8, device="cuda")
    st = L.call("launch_route_plan_noalloc", _request(ids_d, wts_d, outs, 4, 2, 8, ws))
    assert st.code == abi.INVALID_ARGUMENT and b"workspace" in st.message
    # 8192 tokens x 1024 experts needs 1.5 MiB of masks and bases
    st = L.call("launch_route_plan_noalloc", _request(ids_d, wts_d, outs, 8192, 8, 1024))
    assert st.code == abi.INVALID_ARGUMENT and b"scratch" in st.message
    st = L.call("launch_route_plan_noalloc", _request(ids_d, wts_d, outs, 4, 33, 8))
    assert st.code == abi.INVALID_ARGUMENT
    torch.cuda.synchronize()
    assert to_host(outs[0])[0] == 0xFFFFFFFF  # nothing was launched (the -1 fill is intact)


def test_noalloc_graph_replays(eng):
    """Captured once in a HIP graph, replayed three times with new routes
    copied into the captured inputs between replays (eager work and host
    synchronisation in between): every replay equals the workspace entry."""
    import torch

    from pih_amd.device import stream_handle

    tokens, experts, topk = 512, 256, 8
    ids_d = torch.empty(tokens, topk, dtype=torch.int32, device="cuda")
    wts_d = torch.empty(tokens, topk, dtype=torch.float32, device="cuda")
    outs = _outputs(tokens, topk, experts)
    g = torch.cuda.CUDAGraph()
    ids0, wts0 = synth.zipf_router(synth.config_seed(4, 13500), tokens, experts, topk)
    ids_d.copy_(to_dev(ids0))
    wts_d.copy_(to_dev(wts0))
    # one eager call first, as a capturing caller warms up (the pack looks up
    # the device's scratch address on its first call there)
    st = abi.linear_pack().call("launch_route_plan_noalloc", _request(ids_d, wts_d, outs, tokens, topk, experts))
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        req = _request(ids_d, wts_d, outs, tokens, topk, experts, stream=stream_handle())
        st = abi.linear_pack().call("launch_route_plan_noalloc", req)
    assert st.code == abi.OK, st
    for rep in range(3):
        ids, wts = synth.zipf_router(synth.config_seed(4, 13600 + rep), tokens, experts, topk)
        ids_d.copy_(to_dev(ids))
        wts_d.copy_(to_dev(wts))
        torch.cuda.synchronize()
        g.replay()
        got = _host(outs)
        _same(got, _plan(False, ids, wts, experts))
