"""Pre-quantized int4 checkpoints and a persistent prepared-weight format.

The reference quantizes every int4 weight lazily, per process, with RTN
(src/torchinferno/kernels/marlin.py:108-131, called from the Llama3 layer's
``_marlin_proj``, models/llama3/tensor_parallel.py:2732-2794).  This module adds
the two ways around that:

* ``from_gptq`` ingests a GPTQ-style 4-bit checkpoint -- ``qweight`` int32
  ``[K/8, N]`` (eight K rows per word, row 8r+i in bits 4i..4i+3), ``scales``
  ``[K/G, N]``, ``qzeros`` int32 ``[K/G, N/8]`` (eight columns per word) and the
  optional act-order ``g_idx [K]`` -- into the kernel layout.  GPTQ's "v1"
  serialization stores ``zero - 1``, which ``zero_offset`` accounts for.  With
  act-order the K rows are regrouped once at load (each group's 128 rows made
  contiguous) and the matching permutation is applied to the activation's
  columns on every call.
* ``from_awq`` unpacks AWQ's ``[K, N/8]`` words (column order 0,2,4,6,1,3,5,7
  within a word) the same way.
* Zero points.  The GEMM kernels compute the symmetric weight ``(q - 8) * s``.
  Where a checkpoint's zero points z differ from 8 (AWQ, asymmetric GPTQ), the
  weight is ``(q - z) * s = (q - 8) * s + (8 - z) * s``: the prepared weight keeps
  the per-(group, column) offset ``(8 - z) * s`` (fp32, exact), and ``mm`` adds
  its product with the activation's group sums after the GEMM
  (``ti_w4a16_zero_point_add``).
* ``save_prepared`` / ``load_prepared`` keep prepared weights on disk
  (safetensors), so a process loads the kernel layout instead of re-quantizing.

Group size 128 and 4 bits only (the kernels' format).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from .. import _lib
from . import int4 as _int4

_AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)  # AWQ: logical column of nibble slot j is _AWQ_ORDER[j]


@dataclass(frozen=True)
class PreparedInt4:
    """An int4 weight in the kernel layout plus the act-order permutation."""

    q_weight: Tensor          # kernel layout (int32)
    scales: Tensor            # kernel layout (fp16 / bf16, the activation dtype)
    size_k: int
    size_n: int
    perm: Tensor | None = None  # int64 [K]: activation column j of the regrouped problem is a[:, perm[j]]
    zero_offset: Tensor | None = None  # fp32 [K/128, N] = (8 - z) * s; None for symmetric weights

    def mm(self, a: Tensor, workspace: Tensor | None = None, *, out: Tensor | None = None) -> Tensor:
        """a [M, K] @ W -> [M, N] (``int4_mm`` after the act-order gather, if any,
        then the zero-point term for asymmetric weights)."""
        if self.perm is not None:
            a = a.index_select(-1, self.perm).contiguous()
        y = _int4.int4_mm(a, self.q_weight, self.scales, workspace, self.size_n, self.size_k, out=out)
        if self.zero_offset is not None:
            a2 = a.reshape(-1, self.size_k).contiguous()
            _lib.call("ti_w4a16_zero_point_add", a2.data_ptr(), _lib.dtype_code(a2.dtype),
                      self.zero_offset.data_ptr(), y.data_ptr(), a2.size(0), self.size_n, self.size_k,
                      _lib.stream_of(a2))
        return y


def _unpack_words_k(qweight: Tensor) -> Tensor:
    """[K/8, N] int32 -> codes [K, N] (row 8r+i from bits 4i..4i+3)."""
    w = qweight.to(torch.int64) & 0xFFFFFFFF
    shifts = (4 * torch.arange(8, device=w.device, dtype=torch.int64)).view(1, 8, 1)
    return ((w.unsqueeze(1) >> shifts) & 0xF).reshape(-1, w.size(1))


def _unpack_words_n(words: Tensor, order: tuple[int, ...] | None = None) -> Tensor:
    """[R, N/8] int32 -> [R, N]: column 8c+j from nibble slot j (or order[j]'s slot)."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = (4 * torch.arange(8, device=w.device, dtype=torch.int64)).view(1, 1, 8)
    nib = (w.unsqueeze(-1) >> shifts) & 0xF  # [R, N/8, slot]
    if order is not None:
        logical = torch.empty_like(nib)
        logical[..., list(order)] = nib
        nib = logical
    return nib.reshape(w.size(0), -1)


def _zero_offset(zeros: Tensor, scales: Tensor, dtype: torch.dtype, device: torch.device) -> Tensor | None:
    """(8 - z) * s in fp32 [K/128, N] (s rounded to the activation dtype first, as
    the kernels read it), or None when every zero point is 8."""
    z = zeros.to(torch.int64)
    if bool((z == _int4.ZERO_POINT).all()):
        return None
    if bool(((z < 0) | (z > 15)).any()):
        raise ValueError("int4 zero points must lie in [0, 15]")
    s = scales.to(device=device, dtype=dtype).float()
    return ((_int4.ZERO_POINT - z).to(device=device, dtype=torch.float32) * s).contiguous()


def _prepare(codes_kn: Tensor, scales: Tensor, perm: Tensor | None, dtype: torch.dtype,
             device: torch.device, zeros: Tensor | None = None) -> PreparedInt4:
    k, n = codes_kn.shape
    if k % _int4.GROUP_SIZE or not _int4.int4_supports_shape(n, k):
        raise ValueError(f"unsupported int4 shape K={k} N={n} (K % 128 == 0, N % 64 == 0)")
    qweight = _int4.pack_int4(codes_kn.to(device))
    q, s = _int4.repack_int4(qweight, scales.to(device=device, dtype=dtype).contiguous())
    zo = None if zeros is None else _zero_offset(zeros, scales, dtype, device)
    return PreparedInt4(q, s, k, n, None if perm is None else perm.to(device), zo)


def from_gptq(qweight: Tensor, scales: Tensor, qzeros: Tensor | None = None, g_idx: Tensor | None = None, *,
              bits: int = 4, group_size: int = 128, zero_offset: int = 1,
              dtype: torch.dtype | None = None, device: torch.device | str | None = None) -> PreparedInt4:
    """GPTQ 4-bit, group-128 checkpoint tensors -> ``PreparedInt4``.

    ``zero_offset`` is added to the stored zero points (1 for the common "v1"
    serialization that stores ``zero - 1``, 0 for "v2").  ``dtype`` is the
    activation dtype the scales are cast to (default: the checkpoint's)."""
    if bits != 4 or group_size != _int4.GROUP_SIZE:
        raise ValueError("only 4-bit, group-size-128 GPTQ checkpoints are supported")
    if qweight.dtype != torch.int32 or qweight.ndim != 2:
        raise ValueError("GPTQ qweight must be int32 [K/8, N]")
    device = torch.device(device) if device is not None else (
        qweight.device if qweight.is_cuda else torch.device("cuda"))
    codes = _unpack_words_k(qweight)  # [K, N]
    k, n = codes.shape
    if scales.shape != (k // group_size, n):
        raise ValueError(f"GPTQ scales must be [K/128, N] = {(k // group_size, n)}")
    zeros = None
    if qzeros is not None:
        if qzeros.shape != (k // group_size, n // 8):
            raise ValueError(f"GPTQ qzeros must be [K/128, N/8] = {(k // group_size, n // 8)}")
        zeros = _unpack_words_n(qzeros) + zero_offset
    perm = None
    if g_idx is not None:
        g = g_idx.to(torch.int64).cpu()
        if g.shape != (k,):
            raise ValueError("g_idx must be [K]")
        if not torch.equal(g, torch.arange(k) // group_size):
            # act-order: regroup rows so group j owns rows [128j, 128j+128)
            if not torch.equal(torch.bincount(g, minlength=k // group_size),
                               torch.full((k // group_size,), group_size)):
                raise ValueError("g_idx must assign exactly group_size rows to every group")
            perm = torch.sort(g, stable=True).indices
            codes = codes.cpu()[perm]
    return _prepare(codes, scales, perm, dtype or scales.dtype, device, zeros)


def from_awq(qweight: Tensor, scales: Tensor, qzeros: Tensor, *, bits: int = 4, group_size: int = 128,
             dtype: torch.dtype | None = None, device: torch.device | str | None = None) -> PreparedInt4:
    """AWQ 4-bit tensors (``qweight [K, N/8]``, ``qzeros [K/128, N/8]``, scales
    ``[K/128, N]``) -> ``PreparedInt4`` with the checkpoint's zero points."""
    if bits != 4 or group_size != _int4.GROUP_SIZE:
        raise ValueError("only 4-bit, group-size-128 AWQ checkpoints are supported")
    if qweight.dtype != torch.int32 or qweight.ndim != 2:
        raise ValueError("AWQ qweight must be int32 [K, N/8]")
    device = torch.device(device) if device is not None else (
        qweight.device if qweight.is_cuda else torch.device("cuda"))
    codes = _unpack_words_n(qweight, _AWQ_ORDER)  # [K, N]
    k, n = codes.shape
    if scales.shape != (k // group_size, n) or qzeros.shape != (k // group_size, n // 8):
        raise ValueError("AWQ scales must be [K/128, N] and qzeros [K/128, N/8]")
    return _prepare(codes, scales, None, dtype or scales.dtype, device, _unpack_words_n(qzeros, _AWQ_ORDER))


def save_prepared(path: str, weights: dict[str, PreparedInt4]) -> None:
    """Write prepared int4 weights (kernel layout) to a safetensors file."""
    from safetensors.torch import save_file
    tensors, meta = {}, {"format": "torchinferno_amd.int4.v1"}
    for name, w in weights.items():
        tensors[f"{name}.q_weight"] = w.q_weight.contiguous().cpu()
        tensors[f"{name}.scales"] = w.scales.contiguous().cpu()
        if w.perm is not None:
            tensors[f"{name}.perm"] = w.perm.contiguous().cpu()
        if w.zero_offset is not None:
            tensors[f"{name}.zero_offset"] = w.zero_offset.contiguous().cpu()
        meta[f"{name}.shape"] = f"{w.size_k},{w.size_n}"
    save_file(tensors, path, metadata=meta)


def load_prepared(path: str, device: torch.device | str = "cuda") -> dict[str, PreparedInt4]:
    """Read a ``save_prepared`` file back onto ``device``."""
    from safetensors import safe_open
    out = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != "torchinferno_amd.int4.v1":
            raise ValueError(f"{path} is not a torchinferno_amd prepared int4 file")
        keys = set(f.keys())
        for key, shape in meta.items():
            if not key.endswith(".shape"):
                continue
            name = key[: -len(".shape")]
            k, n = (int(v) for v in shape.split(","))
            perm = f.get_tensor(f"{name}.perm").to(device) if f"{name}.perm" in keys else None
            zo = f.get_tensor(f"{name}.zero_offset").to(device) if f"{name}.zero_offset" in keys else None
            out[name] = PreparedInt4(f.get_tensor(f"{name}.q_weight").to(device),
                                     f.get_tensor(f"{name}.scales").to(device), k, n, perm, zo)
    return out
