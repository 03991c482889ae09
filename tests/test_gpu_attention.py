"""The attention core (qim_attention) against softmax(Q K^T * scale) V in
float32 on the CPU, on the same bf16 inputs.

Bar: the kernel rounds P to bf16 for the P V product and writes bf16, so the
output is held to rel-Frobenius <= 1e-2 and a max-abs error of 2 % of the
output's largest magnitude, like the GEMM.  Shapes cover ragged query and key
counts (the last 256-query and 64-key blocks partial), two batches with a
cached prefix (T = P + S), Q/K/V as strided views into one fused QKV output,
and large logits (the running-max subtraction).
"""
import pytest
import torch

from qwen_image_accel.kernels import attention, mxfp8
from tests.helpers import bf16_randn, rel_fro

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def reference(q, k, v, scale):
    """(B, S, H, D) bf16 -> float32 softmax attention, computed on the CPU."""
    qf, kf, vf = (x.float().cpu().permute(0, 2, 1, 3) for x in (q, k, v))  # (B, H, N, D)
    w = torch.softmax(torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale, dim=-1)
    return torch.matmul(w, vf).permute(0, 2, 1, 3)


def check(out, ref):
    got = out.float().cpu()
    err = rel_fro(got.numpy(), ref.numpy())
    mx = (got - ref).abs().max().item()
    assert err < 1e-2, err
    assert mx < 0.02 * ref.abs().max().item(), mx


# (1, 64, 1000, 1), (1, 256, 2000, 4) and (2, 520, 1500, 3) run split over key
# ranges (2, 4 and 3 chunks, the last one ragged) and merged.
@pytest.mark.parametrize("b,s,t,h,mag", [(1, 300, 300, 2, 1.0), (2, 256, 333, 3, 1.0), (1, 64, 1000, 1, 1.0),
                                         (1, 520, 520, 2, 8.0), (1, 256, 2000, 4, 1.0), (2, 520, 1500, 3, 4.0)])
def test_attention_packed(dev, b, s, t, h, mag):
    say("attention", b, s, t, h, mag)
    g = torch.Generator().manual_seed(b * 1000 + s + t + h)
    q = (bf16_randn(g, (b, s, h, 128)) * mag).to(torch.bfloat16).to(dev)
    k = bf16_randn(g, (b, t, h, 128)).to(dev)
    v = bf16_randn(g, (b, t, h, 128)).to(dev)
    scale = 128 ** -0.5
    out = attention.attention(q, k, v)
    torch.cuda.synchronize()
    check(out, reference(q, k, v, scale))


@pytest.mark.parametrize("b", [1, 2])
def test_attention_block_shape_with_split_tail(dev, b):
    """The 1024^2 block's shape (S = T = 4352, 24 heads), as views of a fused
    QKV output.  One image: 408 work items on 256 CUs, one whole round and the
    last 152 items split into 3 key chunks; two images: 816 items, three whole
    rounds and the last 48 items split into 5 chunks.  Checked on heads 0, 11
    and 23 (every query of every image)."""
    s, h = 4352, 24
    say("attention block shape", b, s, h)
    g = torch.Generator().manual_seed(4352)
    qkv = bf16_randn(g, (b, s, 3 * h * 128)).to(dev)
    q, k, v = (qkv[:, :, i * h * 128:(i + 1) * h * 128].unflatten(-1, (h, 128)) for i in range(3))
    out = attention.attention(q, k, v)
    torch.cuda.synchronize()
    for hh in (0, 11, 23):
        sl = slice(hh, hh + 1)
        check(out[:, :, sl], reference(q[:, :, sl], k[:, :, sl], v[:, :, sl], 128 ** -0.5))


def test_attention_on_fused_qkv_views(dev):
    """Q, K, V as column blocks of one (B, S, 3HD) projection (token stride 3HD)."""
    b, s, h = 1, 384, 4
    say("attention qkv views", b, s, h)
    g = torch.Generator().manual_seed(5)
    qkv = bf16_randn(g, (b, s, 3 * h * 128)).to(dev)
    q, k, v = (qkv[:, :, i * h * 128:(i + 1) * h * 128].unflatten(-1, (h, 128)) for i in range(3))
    out = attention.attention(q, k, v, scale=0.1)
    torch.cuda.synchronize()
    check(out, reference(q, k, v, 0.1))


@pytest.mark.parametrize("jump", [30.0, 400.0])
def test_attention_score_jump_past_first_block(dev, jump):
    """Keys whose scores exceed the scores of the first 32 keys by about
    `jump` (natural-log units).  The kernel's first pass keeps each query's
    reference max from its first key sub-block: a jump of 30 stays within
    its range (P up to ~e^33, l and O finite), one of 400 overflows it, which
    the kernel detects and redoes in the running-max form.  Either way the
    output equals the reference."""
    b, s, t, h = 1, 256, 700, 2
    say("attention score jump", jump)
    g = torch.Generator().manual_seed(int(jump))
    # Head 0: every query is q0 plus a little noise; keys 600..609 are q0
    # scaled to a logit of about `jump` against it.
    q0 = bf16_randn(g, (128,)).float()
    q = (q0 + 0.05 * bf16_randn(g, (b, s, h, 128)).float()).to(torch.bfloat16)
    k = bf16_randn(g, (b, t, h, 128))
    v = bf16_randn(g, (b, t, h, 128))
    scale = 128 ** -0.5
    k[0, 600:610, 0] = (q0 * (jump / (scale * q0.square().sum().item()))).to(torch.bfloat16)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    out = attention.attention(q, k, v)
    torch.cuda.synchronize()
    ref = reference(q, k, v, scale)
    assert torch.isfinite(out.float()).all()
    check(out, ref)


# (2, 200, 333, 3): 400 rows, padded to 512, past the last query block's end;
# (1, 256, 2000, 4), (2, 520, 1500, 3) and the 4352 shapes run split and merged.
@pytest.mark.parametrize("b,s,t,h,tiled", [(1, 300, 300, 2, True), (2, 200, 333, 3, False),
                                           (1, 256, 2000, 4, True), (2, 520, 1500, 3, False),
                                           (1, 4352, 4352, 24, True), (2, 4352, 4352, 24, True)])
def test_attention_mxfp8_equals_quantized_output(dev, b, s, t, h, tiled):
    """The fused MXFP8 output is bit-identical to quantizing the bf16 output
    (every code and scale byte, padding rows included: the buffers start
    as 0xff)."""
    say("attention mxfp8", b, s, t, h, tiled)
    g = torch.Generator().manual_seed(7 * b + s + t + h)
    q = bf16_randn(g, (b, s, h, 128)).to(dev)
    kv = bf16_randn(g, (b, t, 2 * h * 128)).to(dev)
    k, v = (kv[:, :, i * h * 128:(i + 1) * h * 128].unflatten(-1, (h, 128)) for i in (0, 1))
    ref = mxfp8.quantize(attention.attention(q, k, v).reshape(b * s, h * 128), tiled=tiled)
    out = mxfp8.empty_quantized(b * s, h * 128, dev, tiled=tiled)
    out.values.view(torch.uint8).fill_(0xff)
    out.scales.view(torch.uint8).fill_(0xff)
    got = attention.attention_mxfp8(q, k, v, tiled=tiled, out=out)
    torch.cuda.synchronize()
    assert torch.equal(got.values.view(torch.uint8), ref.values.view(torch.uint8))
    assert torch.equal(got.scales.view(torch.uint8), ref.scales.view(torch.uint8))


def test_attention_rejects_other_head_dims(dev):
    from qwen_image_accel import _native
    x = torch.zeros(1, 8, 1, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(_native.Unsupported):
        attention.attention(x, x, x)
