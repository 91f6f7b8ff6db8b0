"""NF4 quantisation with double-quantised absmax (the model-load step, not the training hot path).

The reference receives its NF4 weights from bitsandbytes 0.50.2 (``Params4bit._quantize``,
solution/hostload.py:496-524; layout read back in ``_extract_bnb_nf4``, hostload.py:65-96).
bitsandbytes is not part of this build, so this module restates its published algorithm in torch
(runs on whatever device the weight is on):

* ``quantize_4bit(nf4, blocksize=64, compress_statistics=True)``: per block of 64 elements,
  absmax = max|w|, codes = nearest NF4 level of w * (1/absmax), two codes per byte with the even
  element in the high nibble;
* double quantisation: offset = mean(absmax); absmax - offset is quantised blockwise (256 blocks
  per super-block) to 8-bit indices into the signed dynamic map of ``create_dynamic_map``.

Dequantisation parity does not depend on these choices (code2, absmax2 and offset are inputs of
the dequant kernel); agreement with bitsandbytes' own byte output is not checked here.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

# NF4 levels in code order (QLoRA; same table as solution/kernels.py:76-83).
NF4_LEVELS = (
    -1.0,
    -0.6961928009986877,
    -0.5250730514526367,
    -0.39491748809814453,
    -0.28444138169288635,
    -0.18477343022823334,
    -0.09105003625154495,
    0.0,
    0.07958029955625534,
    0.16093020141124725,
    0.24611230194568634,
    0.33791524171829224,
    0.44070982933044434,
    0.5626170039176941,
    0.7229568362236023,
    1.0,
)


def create_dynamic_map(signed: bool = True, max_exponent_bits: int = 7, total_bits: int = 8) -> torch.Tensor:
    """The 8-bit dynamic quantisation map of bitsandbytes (sorted, 256 float32 values): for each
    exponent i, the midpoints of a linear grid on [0.1, 1] scaled by 10^(i - (E-1)), both signs,
    plus 0 and 1."""
    data: list[float] = []
    non_sign_bits = total_bits - 1
    additional_items = 2 ** (non_sign_bits - max_exponent_bits) - 1
    for i in range(max_exponent_bits):
        n = int(2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed
                else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1)
        bounds = torch.linspace(0.1, 1, n, dtype=torch.float32)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        scale = 10 ** (-(max_exponent_bits - 1) + i)
        data += (scale * means).tolist()
        if signed:
            data += (-scale * means).tolist()
    if additional_items > 0:
        bounds = torch.linspace(0.1, 1, additional_items + 1, dtype=torch.float32)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        scale = 10 ** (-(max_exponent_bits - 1) + max_exponent_bits - 1)
        data += (scale * means).tolist()
        if signed:
            data += (-scale * means).tolist()
    data.append(0.0)
    data.append(1.0)
    data += [0.0] * (2**total_bits - len(data))
    data.sort()
    return torch.tensor(data, dtype=torch.float32)


def _nearest(levels_sorted: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Index of the nearest level; a value exactly between two levels takes the lower one."""
    mids = (levels_sorted[:-1] + levels_sorted[1:]) / 2.0
    return torch.bucketize(v, mids, right=False)


def quantize_blockwise(x: torch.Tensor, code: torch.Tensor, blocksize: int) -> tuple[torch.Tensor, torch.Tensor]:
    """8-bit blockwise quantisation of a 1-D float32 tensor: returns (uint8 indices, absmax per
    block)."""
    n = x.numel()
    nb = -(-n // blocksize)
    pad = nb * blocksize - n
    xb = torch.nn.functional.pad(x.reshape(-1).float(), (0, pad)).view(nb, blocksize)
    absmax = xb.abs().amax(dim=1)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    normed = xb * inv[:, None]
    q = _nearest(code.to(x.device), normed).to(torch.uint8).reshape(-1)[:n]
    return q, absmax


@dataclass
class NF4Weight:
    """One NF4 double-quantised matrix in the layout the dequant kernel consumes."""

    packed: torch.Tensor  # uint8 [n/2]
    absmax: torch.Tensor  # uint8 [ceil(n/blocksize)]
    code2: torch.Tensor  # float32 [256]
    absmax2: torch.Tensor  # float32 [ceil(n_blocks/super_blocksize)]
    offset: float
    shape: tuple[int, int]
    blocksize: int = 64
    super_blocksize: int = 256
    extra: dict = field(default_factory=dict)

    def to(self, device) -> "NF4Weight":
        return NF4Weight(self.packed.to(device), self.absmax.to(device), self.code2.to(device),
                         self.absmax2.to(device), self.offset, self.shape, self.blocksize,
                         self.super_blocksize, dict(self.extra))


def quantize_nf4(w: torch.Tensor, blocksize: int = 64, super_blocksize: int = 256) -> NF4Weight:
    """NF4 + double-quant of a 2-D weight (fp16/bf16/fp32), on the weight's device."""
    if w.dim() != 2:
        raise ValueError("quantize_nf4 expects a 2-D weight")
    n = w.numel()
    if n % 2:
        raise ValueError("quantize_nf4: element count must be even")
    dev = w.device
    x = w.reshape(-1).float()
    nb = -(-n // blocksize)
    pad = nb * blocksize - n
    xb = torch.nn.functional.pad(x, (0, pad)).view(nb, blocksize)
    absmax = xb.abs().amax(dim=1)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    normed = (xb * inv[:, None]).reshape(-1)[:n]
    levels = torch.tensor(NF4_LEVELS, dtype=torch.float32, device=dev)
    codes = _nearest(levels, normed).to(torch.uint8)
    packed = (codes[0::2] << 4) | codes[1::2]
    offset = absmax.mean()
    code2 = create_dynamic_map(signed=True).to(dev)
    qabs, absmax2 = quantize_blockwise(absmax - offset, code2, super_blocksize)
    return NF4Weight(packed.contiguous(), qabs.contiguous(), code2, absmax2.float().contiguous(),
                     float(offset.item()), (int(w.shape[0]), int(w.shape[1])), blocksize,
                     super_blocksize)


def concat_segments(parts: list[NF4Weight]) -> tuple[NF4Weight, tuple[int, int], tuple[float, float, float], tuple[int, int]]:
    """Concatenates 1..3 NF4 matrices with equal in_features into one fused segment (the
    [q|k|v] / [gate|up] layout of solution/hostload.py:159-235). Returns (fused weight, split
    bytes, per-segment offsets, absmax2 segment bases)."""
    if not 1 <= len(parts) <= 3:
        raise ValueError("1..3 segments")
    in_f = parts[0].shape[1]
    if any(p.shape[1] != in_f for p in parts):
        raise ValueError("segments must share in_features")
    if any(p.blocksize != parts[0].blocksize or p.super_blocksize != parts[0].super_blocksize for p in parts):
        raise ValueError("segments must share block sizes")
    nbytes = [p.packed.numel() for p in parts]
    hb = parts[0].blocksize // 2
    if any(b % hb for b in nbytes[:-1]):
        raise ValueError("every segment but the last must hold whole absmax blocks")
    splits = [sum(nbytes[: i + 1]) for i in range(len(parts) - 1)]
    total = sum(nbytes)
    while len(splits) < 2:
        splits.append(total)
    n2 = [p.absmax2.numel() for p in parts]
    bases = [sum(n2[: i + 1]) for i in range(len(parts) - 1)]
    while len(bases) < 2:
        bases.append(sum(n2))
    offs = [p.offset for p in parts]
    while len(offs) < 3:
        offs.append(offs[-1])
    fused = NF4Weight(
        torch.cat([p.packed for p in parts]),
        torch.cat([p.absmax for p in parts]),
        parts[0].code2,
        torch.cat([p.absmax2 for p in parts]),
        offs[0],
        (sum(p.shape[0] for p in parts), in_f),
        parts[0].blocksize,
        parts[0].super_blocksize,
    )
    return fused, (splits[0], splits[1]), (offs[0], offs[1], offs[2]), (bases[0], bases[1])
