"""mqc_ssm_fused_fwd_chunked_noalloc (the chunked SSM walk with the library's
fixed device scratch instead of a caller's workspace) against
mqc_ssm_fused_fwd_chunked on the same inputs, through the C ABI: two calls in
a row, the second smaller, and a request beyond the scratch refused."""
import ctypes

import pytest
import torch

from conftest import assert_close

from mambaqc_amd import _native as nat

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(b, T, d, k, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, device=DEV)
    bf = torch.bfloat16
    delta = torch.nn.functional.softplus(r(b, T, d) - 2).to(bf)
    s = r(b, T, d).to(bf)
    Bm = (r(b, T, d, k, 4) * 0.1).to(bf)
    C = (r(b, T, d, k, 4) * 0.1).to(bf)
    la = r(d, k) * 0.5 + 1
    li = r(d, k, 3) * 0.1
    D = torch.ones(d, device=DEV)
    h0 = r(b, d, k, 4) * 0.3
    return delta, s, Bm, C, la, li, D, h0


def _run(lib, name, ins, L, with_ws):
    delta, s, Bm, C, la, li, D, h0 = ins
    b, T, d, k, _ = Bm.shape
    y = torch.empty(b, T, d, 4, device=DEV, dtype=Bm.dtype)
    h = torch.empty(b, d, k, 4, device=DEV, dtype=torch.float32)
    ptrs = [t.data_ptr() for t in (delta, s, Bm, C, la, li, D, h0, y, h)]
    stream = torch.cuda.current_stream().cuda_stream
    tail = []
    if with_ws:
        nbytes = lib.mqc_ssm_chunked_workspace_bytes(b, T, d, k, L)
        ws = torch.empty(max(nbytes, 16), device=DEV, dtype=torch.uint8)
        tail = [ws.data_ptr(), nbytes]
    st = getattr(lib, name)(*ptrs, b, T, d, k, L, 1e-6, nat.BF16, *tail, stream)
    assert st == 0, (name, st, nat.status_string(st))
    torch.cuda.synchronize()
    return y, h


def test_noalloc_matches_workspace_entry_point():
    lib = nat.load()
    assert lib.mqc_ssm_chunked_scratch_bytes() == 32 << 20
    # First call: 8 chunks over 6.3 MB of transitions; second: smaller (3
    # chunks, fewer states), which reuses the scratch the first call filled.
    for shape, L in (((2, 512, 256, 64), 64), ((1, 200, 96, 32), 70)):
        print(f"noalloc case {shape} L={L}", flush=True)
        ins = _inputs(*shape, seed=sum(shape))
        y_ws, h_ws = _run(lib, "mqc_ssm_fused_fwd_chunked", ins, L, True)
        y_na, h_na = _run(lib, "mqc_ssm_fused_fwd_chunked_noalloc", ins, L, False)
        # Same kernels and the same arithmetic: identical results.
        assert torch.equal(y_na, y_ws), f"y differs at {shape}"
        assert torch.equal(h_na, h_ws), f"h_last differs at {shape}"
        y_whole, _ = _run(lib, "mqc_ssm_fused_fwd_chunked", ins, shape[1], True)
        assert_close(y_na, y_whole, 2e-2, f"noalloc vs whole walk {shape}")


def test_noalloc_replays_in_a_hip_graph():
    """The use the entry point is for: captured into a HIP graph (after
    mqc_ssm_noalloc_prepare, so the capture records kernel launches only) and
    replayed, with eager work between the replays, each replay equal to the
    workspace entry point on the same inputs."""
    lib = nat.load()
    assert lib.mqc_ssm_noalloc_prepare() == 0
    b, T, d, k, L = 1, 384, 128, 64, 64
    print(f"noalloc graph case {(b, T, d, k)} L={L}", flush=True)
    ins = _inputs(b, T, d, k, seed=11)
    y_ws, h_ws = _run(lib, "mqc_ssm_fused_fwd_chunked", ins, L, True)
    delta, s, Bm, C, la, li, D, h0 = ins
    y = torch.empty(b, T, d, 4, device=DEV, dtype=Bm.dtype)
    h = torch.empty(b, d, k, 4, device=DEV, dtype=torch.float32)
    ptrs = [t.data_ptr() for t in (delta, s, Bm, C, la, li, D, h0, y, h)]
    graph = torch.cuda.CUDAGraph()
    status = []
    with torch.cuda.graph(graph):
        stream = torch.cuda.current_stream().cuda_stream
        status.append(lib.mqc_ssm_fused_fwd_chunked_noalloc(*ptrs, b, T, d, k, L, 1e-6,
                                                            nat.BF16, stream))
    assert status == [0], status
    for rep in range(3):
        y.fill_(float("nan"))
        h.fill_(float("nan"))
        # Eager use of the same scratch between replays (another shape).
        _run(lib, "mqc_ssm_fused_fwd_chunked_noalloc", _inputs(2, 200, 64, 32, seed=rep), 70,
             False)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_ws), f"replay {rep}: y differs"
        assert torch.equal(h, h_ws), f"replay {rep}: h_last differs"


def test_noalloc_refuses_more_than_its_scratch():
    lib = nat.load()
    b, T, d, k, L = 4, 4096, 2048, 64, 64
    assert lib.mqc_ssm_chunked_workspace_bytes(b, T, d, k, L) > lib.mqc_ssm_chunked_scratch_bytes()
    fake = ctypes.c_void_p(4096)  # never dereferenced: the size check comes first
    st = lib.mqc_ssm_fused_fwd_chunked_noalloc(*[fake] * 7, None, fake, None, b, T, d, k, L,
                                               1e-6, nat.BF16, None)
    assert st == -6, st
