"""Sign-word packing on the host, for tensors that live on the CPU.

The reference's packers are device-agnostic torch (``kernel/utils.py:51-284``) and its loader
expands a checkpoint's words on the CPU (``utils/load_utils.py:392``), so a CPU tensor is packed
here, on the CPU, into the words the HIP kernels of ``csrc/nq_pack.hip`` write for the same input,
bit for bit. CUDA tensors never come here, and these functions never stand in for a GPU path.

Every layout is a bijection between the elements of a block and the bits of its words, so each
function gathers a block's sign bits into bit order (bit b of a word takes the element whose
position is b) and lets ``numpy.packbits(bitorder="little")`` build the little-endian words, eight
bits per byte; unpacking runs the same gather backwards on ``numpy.unpackbits``. A value packs as
-1 (bit set) iff it is negative. Rows go in chunks so that the boolean temporaries stay small.
"""
from __future__ import annotations

import numpy as np
import torch

_ROWS_PER_CHUNK = 4096

# bit position of element e (0..31) of a 32-column block, per method code (0 lsb_first, 1 half2)
_POSITION = {0: np.arange(32), 1: np.array([15 - e // 2 + 16 * (e % 2) for e in range(32)])}
# the element each bit position takes (the inverse permutation)
_ELEMENT = {code: np.argsort(pos) for code, pos in _POSITION.items()}


def _marlin_tile_gather() -> np.ndarray:
    """For one Marlin tile (64 outputs x 16 reductions, 32 words of 32 bits): entry 32 w + b is the
    flat index o * 16 + k (o < 64, k < 16) of the element at bit b of the tile's word w. Element
    (o, k) sits in word 4 (o % 8) + (k % 8) / 2 at bit 15 - 2 ((o % 16) / 8) - k / 8 + 16 (k % 2)
    - 4 (o / 16) (kernel/utils.py:192-205)."""
    o = np.arange(64)[:, None]
    k = np.arange(16)[None, :]
    word = 4 * (o % 8) + (k % 8) // 2
    bit = 15 - 2 * ((o % 16) // 8) - k // 8 + 16 * (k % 2) - 4 * (o // 16)
    gather = np.empty(1024, dtype=np.int64)
    gather[(32 * word + bit).reshape(-1)] = (o * 16 + k).reshape(-1)
    return gather


_MARLIN_GATHER = _marlin_tile_gather()


def _words_from_bits(bits: np.ndarray) -> np.ndarray:
    """bool [..., 32] in bit order -> uint32 [...]."""
    packed = np.packbits(np.ascontiguousarray(bits), axis=-1, bitorder="little")
    return packed.view("<u4")[..., 0]


def _bits_from_words(words: np.ndarray) -> np.ndarray:
    """32-bit words [...] (int32 or uint32, little-endian) -> uint8 0/1 [..., 32] in bit order."""
    words = np.ascontiguousarray(words)
    assert words.dtype.itemsize == 4, words.dtype
    return np.unpackbits(words.view(np.uint8).reshape(*words.shape, 4), axis=-1, bitorder="little")


def _blocks(neg: np.ndarray, words: int) -> np.ndarray:
    """bool [n, cols] -> bool [n, words, 32], clear (+1) past ``cols``."""
    out = np.zeros((neg.shape[0], words * 32), dtype=bool)
    out[:, :neg.shape[1]] = neg
    return out.reshape(neg.shape[0], words, 32)


def pack_signs(signs: torch.Tensor, method: int) -> torch.Tensor:
    """int8 [R, C] -> int32 words [R, ceil(C/32)] in ``method`` bit order (as ``nq_pack_signs``)."""
    src = signs.detach().contiguous().numpy()
    n_rows, n_cols = src.shape
    words = (n_cols + 31) // 32
    out = np.empty((n_rows, words), dtype=np.uint32)
    order = _ELEMENT[method]
    for r0 in range(0, n_rows, _ROWS_PER_CHUNK):
        bits = _blocks(src[r0:r0 + _ROWS_PER_CHUNK] < 0, words)
        out[r0:r0 + _ROWS_PER_CHUNK] = _words_from_bits(bits[:, :, order])
    return torch.from_numpy(out.view(np.int32))


def _element_bits(words: np.ndarray, n_cols: int, method: int) -> np.ndarray:
    """uint8 0/1 [n, n_cols]: element j's sign bit of word rows [n, ceil(n_cols/32)]."""
    bits = _bits_from_words(words)[:, :, _POSITION[method]]
    return bits.reshape(words.shape[0], -1)[:, :n_cols]


def unpack_signs(packed: torch.Tensor, n_rows: int, n_cols: int, method: int) -> torch.Tensor:
    """Inverse of :func:`pack_signs`: int8 {-1, +1} [R, C] (as ``nq_unpack_signs``)."""
    words = packed.detach().contiguous().numpy()
    out = np.empty((n_rows, n_cols), dtype=np.int8)
    for r0 in range(0, n_rows, _ROWS_PER_CHUNK):
        bits = _element_bits(words[r0:r0 + _ROWS_PER_CHUNK], n_cols, method)
        out[r0:r0 + _ROWS_PER_CHUNK] = 1 - 2 * bits.astype(np.int8)
    return torch.from_numpy(out)


def repack_signs(packed: torch.Tensor, n_rows: int, n_cols: int, src: int, dst: int) -> torch.Tensor:
    """Words in ``src`` order -> the words ``pack_signs`` makes in ``dst`` order from the same signs
    (padding bits cleared), as ``nq_repack_signs``."""
    words = packed.detach().contiguous().numpy()
    n_words = words.shape[1]
    out = np.empty((n_rows, n_words), dtype=np.uint32)
    order = _ELEMENT[dst]
    for r0 in range(0, n_rows, _ROWS_PER_CHUNK):
        bits = _blocks(_element_bits(words[r0:r0 + _ROWS_PER_CHUNK], n_cols, src).astype(bool), n_words)
        out[r0:r0 + _ROWS_PER_CHUNK] = _words_from_bits(bits[:, :, order])
    return torch.from_numpy(out.view(np.int32))


def _marlin_words(neg: np.ndarray) -> np.ndarray:
    """bool sign bits [O, K] (O % 64 == 0, K % 16 == 0) -> uint32 Marlin words [K/16, O/2]."""
    O, K = neg.shape
    tiles = neg.reshape(O // 64, 64, K // 16, 16).transpose(2, 0, 1, 3).reshape(K // 16, O // 64, 1024)
    bits = tiles[:, :, _MARLIN_GATHER].reshape(K // 16, O // 64, 32, 32)
    return _words_from_bits(bits).reshape(K // 16, O // 2)


def pack_marlin(weight: torch.Tensor) -> torch.Tensor:
    """{-1, +1} [O, K] -> int32 Marlin words [K/16, O/2] (as ``nq_pack_marlin``)."""
    w = weight.detach().contiguous()
    neg = (w < 0).numpy()
    return torch.from_numpy(_marlin_words(neg).view(np.int32))


def repack_marlin(packed: torch.Tensor, O: int, K: int, O_pad: int, K_pad: int, src: int) -> torch.Tensor:
    """Sign words of [O, K] in ``src`` order -> Marlin words of the matrix padded with +1 to
    [O_pad, K_pad] (as ``nq_repack_marlin``)."""
    words = packed.detach().contiguous().numpy()
    neg = np.zeros((O_pad, K_pad), dtype=bool)
    for r0 in range(0, O, _ROWS_PER_CHUNK):
        r1 = min(r0 + _ROWS_PER_CHUNK, O)
        neg[r0:r1, :K] = _element_bits(words[r0:r1], K, src).astype(bool)
    return torch.from_numpy(_marlin_words(neg).view(np.int32))


def permute_marlin_scales(s_in: torch.Tensor, s_out: torch.Tensor):
    """The Marlin scale orders (as ``nq_permute_marlin_scales``): natural input index 16c + 8a +
    2b + d at 16c + 4b + 2a + d, natural output index 32c + 8a + 2b + d at 32c + 8b + 2a + d
    (kernel/utils.py:206-209)."""
    p_in = s_in.reshape(-1, 2, 4, 2).transpose(1, 2).reshape(-1).contiguous()
    p_out = s_out.reshape(-1, 4, 4, 2).transpose(1, 2).reshape(-1).contiguous()
    return p_in, p_out
