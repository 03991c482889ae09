"""3-axis (frame, height, width) RoPE table of the joint text/image sequence.

Host-side input construction for the RoPE kernels, following
QwenImage21Rope (WHL!diffusers/models/transformers/transformer_qwenimage21.py:
652-710): text tokens advance one shared position on all three axes; an image
block freezes the frame axis at the position reached after the text and lays
its tokens on a height/width grid centred on zero.  Each axis of width d
contributes d/2 complex entries polar(1, pos * theta^(-2i/d)), computed in fp32
on the CPU like the reference.
"""
import torch


def positions(text_tokens, frames, height, width):
    """(S, 3) int64 positions of `text_tokens` text tokens followed by one
    frames x height x width image block."""
    rows = [(t, t, t) for t in range(text_tokens)]
    for _ in range(frames):
        for h in range(-(height - height // 2), height // 2):
            for w in range(-(width - width // 2), width // 2):
                rows.append((text_tokens, h, w))
    return torch.tensor(rows, dtype=torch.int64)


def freqs(pos, dims=(16, 56, 56), theta=10000):
    """(S, sum(dims)/2) complex64 table for positions `pos` (S, 3)."""
    cols = []
    for axis, dim in enumerate(dims):
        inv = 1.0 / torch.pow(theta, torch.arange(0, dim, 2).to(torch.float32).div(dim))
        angle = torch.outer(pos[:, axis].to(torch.float32), inv)
        cols.append(torch.polar(torch.ones_like(angle), angle))
    return torch.cat(cols, dim=-1)


def image_table(text_tokens, height, width, device=None, dims=(16, 56, 56), theta=10000):
    """Table of `text_tokens` text tokens + one height x width image."""
    f = freqs(positions(text_tokens, 1, height, width), dims, theta)
    return f if device is None else f.to(device)
