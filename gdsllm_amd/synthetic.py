"""Synthetic weights and activations in the reference's on-disk byte layouts.

The converters (tools/convert_gguf.py:155-185, tools/convert_qwen_moe.py:205-276)
copy GGUF blocks verbatim and pack affine-Q4 as uint32 words + fp16 scales /
biases; these generators produce the same layouts from a seeded
torch.Generator, on whatever device the generator lives on, so a CPU copy and
a GPU copy made from equal seeds hold identical bytes.

Distributions follow the benchmark configurations: Q4_0 d ~ U(0.005, 0.02) and
uniform nibbles; Q8_0 d ~ U(0.001, 0.004) and q ~ U[-127, 127]; per-column
int8 scale ~ U(0.001, 0.004) and q ~ U[-128, 127]; affine
scale ~ U(0.005, 0.02), bias ~ N(0, 0.05), uniform nibbles; x ~ N(0, 1) fp16.
"""

from __future__ import annotations

import torch


def _dev(gen: torch.Generator) -> torch.device:
    return gen.device


def _fp16_uniform(n: int, lo: float, hi: float, gen: torch.Generator) -> torch.Tensor:
    return torch.empty(n, dtype=torch.float32, device=_dev(gen)).uniform_(lo, hi, generator=gen).to(torch.float16)


def q4_0_weights(rows: int, cols: int, gen: torch.Generator, d_range=(0.005, 0.02)) -> torch.Tensor:
    """uint8 [rows, cols/32*18]: row-major GGUF Q4_0 blocks {fp16 d, u8 qs[16]}."""
    if cols % 32:
        raise ValueError("cols must be a multiple of 32")
    nblk = rows * cols // 32
    d = _fp16_uniform(nblk, *d_range, gen)
    qs = torch.randint(0, 256, (nblk, 16), dtype=torch.uint8, device=_dev(gen), generator=gen)
    out = torch.empty(nblk, 18, dtype=torch.uint8, device=_dev(gen))
    out[:, :2] = d.view(torch.uint8).view(nblk, 2)
    out[:, 2:] = qs
    return out.view(rows, cols // 32 * 18)


def q8_0_weights(rows: int, cols: int, gen: torch.Generator, d_range=(0.001, 0.004)) -> torch.Tensor:
    """uint8 [rows, cols/32*34]: row-major GGUF Q8_0 blocks {fp16 d, i8 qs[32]}."""
    if cols % 32:
        raise ValueError("cols must be a multiple of 32")
    nblk = rows * cols // 32
    d = _fp16_uniform(nblk, *d_range, gen)
    qs = torch.randint(-127, 128, (nblk, 32), dtype=torch.int8, device=_dev(gen), generator=gen)
    out = torch.empty(nblk, 34, dtype=torch.uint8, device=_dev(gen))
    out[:, :2] = d.view(torch.uint8).view(nblk, 2)
    out[:, 2:] = qs.view(torch.uint8)
    return out.view(rows, cols // 32 * 34)


def int8_weights(rows: int, cols: int, gen: torch.Generator, s_range=(0.001, 0.004)):
    """(q int8 [rows, cols], scale fp16 [1, cols]): the per-column int8 format
    of tools/convert_weights.py:55-83 with q ~ U[-128, 127] and scale ~ U(s_range)."""
    q = torch.randint(-128, 128, (rows, cols), dtype=torch.int8, device=_dev(gen), generator=gen)
    return q, _fp16_uniform(cols, *s_range, gen).view(1, cols)


def affine_q4_weights(shape, group_size: int, gen: torch.Generator):
    """(words int32 [..., cols/8], scales fp16 [..., cols/g], biases fp16 [..., cols/g]).

    `shape` is the unpacked [..., cols] shape (e.g. [E, N, K] for stacked experts).
    Words are stored as int32 (same bits as the reference's uint32).
    """
    *lead, cols = shape
    if cols % 8 or cols % group_size:
        raise ValueError("cols must be a multiple of 8 and of group_size")
    n_words = 1
    for s in lead:
        n_words *= s
    n_groups = n_words * (cols // group_size)
    n_words *= cols // 8
    words = torch.randint(0, 256, (n_words * 4,), dtype=torch.uint8, device=_dev(gen), generator=gen).view(torch.int32)
    scales = _fp16_uniform(n_groups, 0.005, 0.02, gen)
    biases = (torch.randn(n_groups, dtype=torch.float32, device=_dev(gen), generator=gen) * 0.05).to(torch.float16)
    return (words.view(*lead, cols // 8), scales.view(*lead, cols // group_size), biases.view(*lead, cols // group_size))


def activations(batch: int, cols: int, gen: torch.Generator) -> torch.Tensor:
    """fp16 [batch, cols] ~ N(0, 1)."""
    return torch.randn(batch, cols, dtype=torch.float32, device=_dev(gen), generator=gen).to(torch.float16)


def pack_buffer(parts, align: int = 4096):
    """Concatenate byte tensors into one uint8 tensor, each part at an
    `align`-aligned offset (the layer-file rule, tools/convert_gguf.py:80-89).
    Returns (buffer, [offsets])."""
    offsets, total = [], 0
    for p in parts:
        offsets.append(total)
        total += (p.numel() * p.element_size() + align - 1) // align * align
    dev = parts[0].device if parts else torch.device("cpu")
    buf = torch.zeros(max(total, align), dtype=torch.uint8, device=dev)
    for p, off in zip(parts, offsets):
        b = p.contiguous().view(torch.uint8).reshape(-1)
        buf[off:off + b.numel()] = b
    return buf, offsets
