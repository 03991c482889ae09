"""HIP graphs: the library's launches captured in a graph (as bench.py times
them) and replayed several times, with the program's own eager work and
synchronizations between the replays, give the eager result bit for bit on
every replay.  Covered: MMDiTBlock.forward with the stand-in attention, with
the attention core writing the out-projection's MXFP8 input, and with V^T
written by the QKV projection; and the attention core alone at the config's
own size, where the last round of work items is split over key ranges and
merged (workspace partials written and read inside the graph).
"""
import pytest
import torch

from qwen_image_accel import rope
from qwen_image_accel.block import MMDiTBlock
from qwen_image_accel.kernels import attention
from tests.helpers import bf16_randn

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def replay_checks(fn, ref, replays=4):
    """Capture fn() in a graph and check each replay (and an eager call made
    between replays) against ref."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    for r in range(replays):
        other = fn()                 # eager work of the program itself between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r} differs from the eager result"
        assert torch.equal(other, ref), f"eager call after replay {r - 1} differs"
    del graph


@pytest.mark.parametrize("mode", ["stand_in", "attention_mxfp8", "fused_attention"])
def test_block_graph_replays_equal_eager(dev, mode):
    g = torch.Generator().manual_seed(7)
    dim, heads, ffn, side = 512, 4, 1024, 16
    s = 256 + side * side
    say("block graph", mode, s, dim)
    blk = MMDiTBlock.random(g, dim=dim, heads=heads, ffn=ffn, device=dev)
    h = bf16_randn(g, (1, s, dim)).to(dev)
    mod = bf16_randn(g, (1, 6, dim), 0.5).to(dev)
    freqs = rope.image_table(256, side, side, dev)
    kw = {"stand_in": {}, "attention_mxfp8": {"attention_mxfp8_fn": attention.attention_mxfp8},
          "fused_attention": {"fused_attention": True}}[mode]

    def fwd():
        return blk.forward(h, mod, freqs, **kw)
    ref = fwd()
    torch.cuda.synchronize()
    replay_checks(fwd, ref)


def test_attention_graph_with_split_tail(dev):
    """S = T = 4352, 24 heads (the 1024^2 config): 408 work items on the CUs
    leave a partial last round, which runs as key-range chunks plus the merge."""
    g = torch.Generator().manual_seed(11)
    b, s, h = 1, 4352, 24
    say("attention graph", b, s, h)
    qkv = bf16_randn(g, (b, s, 3, h, 128)).to(dev)
    q, k, v = qkv.unbind(2)

    def run():
        return attention.attention(q, k, v)
    ref = run()
    torch.cuda.synchronize()
    replay_checks(run, ref, replays=3)
