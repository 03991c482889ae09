"""qim_attention_noalloc (the attention core with its workspace in the
library's own device array) against qim_attention with a caller-allocated
workspace, through the C ABI: two calls in a row, the second smaller, so the
second runs over what the first left in the shared array.  Same kernels and
the same work split on both sides, so the outputs are compared bit for bit.
"""
import pytest
import torch

from qwen_image_accel import _native
from tests.helpers import bf16_randn

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _inputs(g, b, s, t, h, dev):
    q = bf16_randn(g, (b, s, h, 128)).to(dev)
    kv = bf16_randn(g, (b, t, 2 * h * 128)).to(dev)          # K and V as column blocks of one tensor
    return q, kv


def _with_workspace(q, kv, b, s, t, h):
    o = torch.empty(b, s, h, 128, dtype=torch.bfloat16, device=q.device)
    nbytes = _native.lib().qim_attention_workspace_bytes(b, s, t, h, 128)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    row = 2 * h * 128
    _native.call("qim_attention", _native.ptr(q), h * 128, _native.ptr(kv), row,
                 ctypes_offset(kv, h * 128), row, _native.ptr(o), h * 128, _native.ptr(ws), nbytes,
                 b, s, t, h, 128, 128 ** -0.5, _native.stream(q.device))
    return o


def _no_alloc(q, kv, b, s, t, h):
    o = torch.full((b, s, h, 128), float("nan"), dtype=torch.bfloat16, device=q.device)
    row = 2 * h * 128
    _native.call("qim_attention_noalloc", _native.ptr(q), h * 128, _native.ptr(kv), row,
                 ctypes_offset(kv, h * 128), row, _native.ptr(o), h * 128, b, s, t, h, 128, 128 ** -0.5,
                 _native.stream(q.device))
    return o


def ctypes_offset(t, elements):
    import ctypes
    return ctypes.c_void_p(t.data_ptr() + elements * t.element_size())


def test_no_alloc_attention_equals_workspace_entry_point(dev):
    g = torch.Generator().manual_seed(2024)
    # One image at 1024^2 (the largest problem the scratch array holds: V^T
    # tiles plus the split tail's partial rows), then a smaller, split one.
    for b, s, t, h in [(1, 4352, 4352, 24), (2, 520, 1500, 3)]:
        say("attention noalloc", b, s, t, h)
        q, kv = _inputs(g, b, s, t, h, dev)
        ref = _with_workspace(q, kv, b, s, t, h)
        got = _no_alloc(q, kv, b, s, t, h)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_no_alloc_attention_rejects_problems_above_its_scratch(dev):
    """S = T = 16640 with 24 heads needs more than the array holds: rejected
    with QIM_ERR_SHAPE before anything is launched."""
    need = _native.lib().qim_attention_workspace_bytes(1, 16640, 16640, 24, 128)
    assert need > (64 << 20)
    say("attention noalloc oversize", need)
    rc = _native.lib().qim_attention_noalloc(16, 3072, 16, 3072, 16, 3072, 16, 3072, 1, 16640, 16640, 24, 128,
                                              0.1, None)
    assert rc == _native.QIM_ERR_SHAPE
    assert b"scratch" in _native.lib().qim_last_error()


def test_no_alloc_attention_under_graph_capture(dev):
    """The use it is for: a call captured in a HIP graph.  The first call on
    the device (made before the capture) resolves the scratch array; the
    captured call then allocates nothing, and every replay, with the
    program's own eager work between replays, equals qim_attention bit for
    bit."""
    g = torch.Generator().manual_seed(77)
    b, s, t, h = 1, 1100, 1300, 6
    say("attention noalloc graph", b, s, t, h)
    q, kv = _inputs(g, b, s, t, h, dev)
    ref = _with_workspace(q, kv, b, s, t, h)
    o = torch.empty(b, s, h, 128, dtype=torch.bfloat16, device=dev)
    row = 2 * h * 128

    def call():
        _native.call("qim_attention_noalloc", _native.ptr(q), h * 128, _native.ptr(kv), row,
                     ctypes_offset(kv, h * 128), row, _native.ptr(o), h * 128, b, s, t, h, 128, 128 ** -0.5,
                     _native.stream(q.device))

    call()                                   # first call on the device: before any capture
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), ref.view(torch.int16))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for r in range(3):
        o.fill_(float("nan"))                # eager work between replays
        other = _with_workspace(q, kv, b, s, t, h)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), ref.view(torch.int16)), f"replay {r}"
        assert torch.equal(other.view(torch.int16), ref.view(torch.int16))
    del graph
