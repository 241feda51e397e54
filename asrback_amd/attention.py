"""Attention ops on the HIP kernels of ``libasrattn.so``.

These take PyTorch tensors (often strided views: heads split out of a fused
projection, slices of a preallocated cache), pass their device pointers and
element strides to the C ABI, and launch on the current HIP stream, so they
can run inside ``torch.cuda.graph`` capture (a hipGraph on ROCm).  Nothing
here synchronizes with the device.

Three entry points cover every attention call of the reference:

* :func:`sdpa` -- ``F.scaled_dot_product_attention`` as the reference calls
  it, on ``(batch, heads, length, head_dim)`` tensors, with the masks it
  builds expressed as key counts (:class:`KeyPrefix`).  Rows with one query
  go to the decode kernel, longer ones to the multi-row kernel.
* :func:`varlen_attn` -- ``torch.nn.attention.varlen.varlen_attn`` with the
  arguments the reference passes (``seqused_k``, ``window_size``,
  ``enable_gqa``, ``num_splits``).
* :func:`decode` -- one query per sequence over a key/value cache, any
  strides (the Whisper ``(B, H, L, D)`` and Qwen3 ``(B, L, H_kv, D)``
  caches).

The fused neighbours of those calls: :func:`flash` (the multi-row kernel
itself), :func:`flash_fsmn` (SenseVoice attention plus its FSMN memory),
:func:`decode_append` (the decoder step with its norms, rotation and cache
write) and :func:`greedy_choice` (argmax and its log-probability).

The reference's masks are all prefix masks: each query row sees keys
``0 .. n-1`` (optionally causal on top).  A boolean mask with a hole is
refused (:meth:`KeyPrefix.from_mask`).

Split-K decode and the split greedy choice keep partials in a workspace the
caller owns: a decoder sizes one buffer at its largest bucket
(:func:`decode_workspace_size`, :func:`choice_workspace_size`) and runs its
steps inside :func:`workspace`; calls outside any take a stream-ordered
temporary.
"""

from __future__ import annotations

import contextlib
import ctypes
import math
import threading
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


@dataclass(frozen=True)
class KeyPrefix:
    """A key mask that shows each row the keys ``0 .. n_b - 1``.

    ``n_b = positions[b] + 1`` (int64 ``positions``, the Whisper decoder step,
    ``whisper.py:263-264``) or ``n_b = lengths[b]`` (int32 ``lengths``, the
    padding masks of ``sensevoice.py:548-550`` and ``qwen3_asr.py:510-515``).
    Both stay on the device, so a captured graph sees their new values on
    every replay.
    """

    positions: Tensor | None = None
    lengths: Tensor | None = None

    def __post_init__(self) -> None:
        if (self.positions is None) == (self.lengths is None):
            raise ValueError("KeyPrefix takes exactly one of positions and lengths")
        if self.positions is not None and self.positions.dtype != torch.int64:
            raise TypeError(f"positions must be int64, got {self.positions.dtype}")
        if self.lengths is not None and self.lengths.dtype != torch.int32:
            raise TypeError(f"lengths must be int32, got {self.lengths.dtype}")

    @classmethod
    def from_mask(cls, mask: Tensor) -> KeyPrefix:
        """The prefix described by a boolean ``(batch, 1, 1, length)`` or
        ``(batch, length)`` mask that is True for keys ``0 .. n_b - 1``.

        A mask with a hole (a False before a True in some row) describes an
        attention the kernels do not compute: it raises ``ValueError``.  The
        check reads the comparison back from the device, so a tensor mask is
        refused during graph capture (pass a :class:`KeyPrefix` there, as
        every module of this package does)."""
        if mask.dtype != torch.bool:
            raise TypeError(f"only boolean prefix masks are supported, got {mask.dtype}")
        if mask.dim() < 2 or mask.numel() != mask.shape[0] * mask.shape[-1]:
            raise ValueError(f"expected a (batch, length) or (batch, 1, 1, length) mask, got {tuple(mask.shape)}")
        if mask.is_cuda and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("a boolean mask cannot be checked during graph capture; pass a KeyPrefix")
        rows = mask.reshape(mask.shape[0], mask.shape[-1])
        lengths = rows.sum(dim=-1, dtype=torch.int32)
        prefix = torch.arange(rows.shape[-1], device=rows.device)[None, :] < lengths[:, None]
        if not torch.equal(rows, prefix):
            raise ValueError("the attention kernels take prefix masks only (row b sees keys 0 .. n_b - 1); "
                             "this mask has a False before a True")
        return cls(lengths=lengths)


@dataclass(frozen=True)
class PageTable:
    """A paged key/value layout for :func:`decode` / :func:`decode_append`:
    the cache tensors are pools ``(num_pages, page_size, heads_kv,
    head_dim)`` and logical page ``i`` of sequence ``b`` (its keys ``i *
    page_size ..``) is pool page ``block_table[b, i]`` (int32 ``(batch,
    pages_per_row)``, on the device; entries outside the pool are skipped).
    ``max_len`` bounds the keys a sequence may use (default: the table's
    reach).  Generalizes the reference's fixed ``row * 1024`` slab
    (``qwen3_asr.py:511-512``)."""

    block_table: Tensor
    max_len: int | None = None

    def __post_init__(self) -> None:
        if self.block_table.dtype != torch.int32 or self.block_table.dim() != 2:
            raise TypeError("block_table must be an int32 (batch, pages_per_row) tensor")
        if self.block_table.stride(-1) != 1:
            raise ValueError("block_table rows must be contiguous")


def _paged(pages: PageTable, k: Tensor, v: Tensor, batch: int) -> tuple[_lib.PagedKV, int]:
    """``asrattn_paged_kv`` for pools ``k``/``v`` and the keys a sequence may use."""
    table = pages.block_table
    if table.shape[0] < batch:
        raise ValueError(f"block_table has {table.shape[0]} rows for {batch} sequences")
    page_size = k.shape[1]
    reach = table.shape[1] * page_size
    max_len = reach if pages.max_len is None else pages.max_len
    if not 0 <= max_len <= reach:
        raise ValueError(f"max_len {max_len} outside the table's reach {reach}")
    pk = _lib.PagedKV()
    pk.block_table = table.data_ptr()
    pk.bt_stride = table.stride(0)
    pk.page_size = page_size
    pk.num_pages = k.shape[0]
    pk.k_page_stride, pk.v_page_stride = k.stride(0), v.stride(0)
    return pk, max_len


def _dtype_code(*tensors: Tensor) -> int:
    dtype = tensors[0].dtype
    if dtype not in _DTYPES:
        raise TypeError(f"attention supports float32 and bfloat16, got {dtype}")
    for tensor in tensors:
        if tensor.dtype != dtype:
            raise TypeError(f"mixed dtypes: {dtype} and {tensor.dtype}")
        if tensor.device.type != "cuda":
            raise RuntimeError(
                f"attention kernels run on the GPU only; got a tensor on {tensor.device}"
            )
    return _DTYPES[dtype]


def _aligned(t: Tensor, dims: tuple[int, ...]) -> Tensor:
    """``t`` itself when its rows can be read with 16-byte vectors, else a
    contiguous copy.  ``dims`` are the strided (non head_dim) axes."""
    per_vec = 16 // t.element_size()
    if (
        t.stride(-1) == 1
        and t.data_ptr() % 16 == 0
        and all(t.stride(d) % per_vec == 0 for d in dims)
    ):
        return t
    return t.contiguous()


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_device(*tensors: Tensor | None) -> torch.device:
    device = None
    for tensor in tensors:
        if tensor is None:
            continue
        if device is None:
            device = tensor.device
        elif tensor.device != device:
            raise RuntimeError(f"tensors on different devices: {device} and {tensor.device}")
    if device.index is not None and device.index != torch.cuda.current_device():
        raise RuntimeError(
            f"tensors are on {device} but the current device is cuda:{torch.cuda.current_device()}"
        )
    return device


def _int32(t: Tensor | None, name: str) -> Tensor | None:
    if t is None:
        return None
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32, got {t.dtype}")
    return t.contiguous()


def _fwd_params(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    out: Tensor | None,
    causal: int,
    cu_seqlens_q: Tensor | None,
    cu_seqlens_k: Tensor | None,
    max_len_q: int | None,
    max_len_k: int | None,
    seqused_k: Tensor | None,
    scale: float | None,
    force_valu: bool,
    window: int = 0,
    flags: int = 0,
) -> tuple[_lib.FwdParams, Tensor, torch.device, tuple]:
    """``asrattn_fwd_params`` for :func:`flash`; returns them with ``out``,
    the device and the tensors the parameters point into (kept alive until
    the launch)."""
    dtype = _dtype_code(q, k, v)
    packed = cu_seqlens_q is not None
    if packed != (cu_seqlens_k is not None):
        raise ValueError("cu_seqlens_q and cu_seqlens_k go together")
    rank = 3 if packed else 4
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dim() != rank:
            raise ValueError(f"{name} must have {rank} dimensions, got shape {tuple(t.shape)}")
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
    head_dim = q.shape[-1]
    heads_q, heads_kv = q.shape[-2], k.shape[-2]
    if k.shape[-1] != head_dim:
        raise ValueError("q and k head_dim differ")
    if heads_q % heads_kv:
        raise ValueError(f"{heads_q} query heads are not a multiple of {heads_kv} kv heads")
    strided = (0, 1, 2) if not packed else (0, 1)
    q, k, v = (_aligned(t, strided) for t in (q, k, v))
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        # The kernels write each head's head_dim elements contiguously.
        raise ValueError("out must match q's shape and dtype, with a unit last stride")
    device = _check_device(q, k, v, out, cu_seqlens_q, cu_seqlens_k, seqused_k)
    cu_seqlens_q = _int32(cu_seqlens_q, "cu_seqlens_q")
    cu_seqlens_k = _int32(cu_seqlens_k, "cu_seqlens_k")
    seqused_k = _int32(seqused_k, "seqused_k")

    params = _lib.FwdParams()
    params.q, params.k, params.v, params.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    if packed:
        if max_len_q is None or max_len_k is None:
            raise ValueError("packed sequences need max_len_q and max_len_k")
        batch = cu_seqlens_q.shape[0] - 1
        if cu_seqlens_k.shape[0] != batch + 1:
            raise ValueError("cu_seqlens_q and cu_seqlens_k have different lengths")
        for prefix, t in (("q", q), ("k", k), ("v", v), ("o", out)):
            setattr(params, f"{prefix}_batch_stride", 0)
            setattr(params, f"{prefix}_token_stride", t.stride(0))
            setattr(params, f"{prefix}_head_stride", t.stride(1))
    else:
        batch = q.shape[0]
        if k.shape[0] != batch:
            raise ValueError("q and k batch sizes differ")
        max_len_q = q.shape[1] if max_len_q is None else max_len_q
        max_len_k = k.shape[1] if max_len_k is None else max_len_k
        if max_len_q > q.shape[1] or max_len_k > k.shape[1]:
            raise ValueError("max_len_q / max_len_k exceed the tensors")
        for prefix, t in (("q", q), ("k", k), ("v", v), ("o", out)):
            setattr(params, f"{prefix}_batch_stride", t.stride(0))
            setattr(params, f"{prefix}_token_stride", t.stride(1))
            setattr(params, f"{prefix}_head_stride", t.stride(2))
    if seqused_k is not None and seqused_k.shape[0] != batch:
        raise ValueError(f"seqused_k has {seqused_k.shape[0]} entries for {batch} sequences")
    params.cu_seqlens_q = _ptr(cu_seqlens_q)
    params.cu_seqlens_k = _ptr(cu_seqlens_k)
    params.seqused_k = _ptr(seqused_k)
    params.batch = batch
    params.heads_q = heads_q
    params.heads_kv = heads_kv
    params.head_dim = head_dim
    params.max_len_q = max_len_q
    params.max_len_k = max_len_k
    params.causal = causal
    params.dtype = dtype
    params.scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    params.flags = flags | (_lib.FWD_FORCE_VALU if force_valu else 0)
    params.window = window or 0
    return params, out, device, (q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k)


def flash(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    out: Tensor | None = None,
    causal: int = _lib.CAUSAL_NONE,
    cu_seqlens_q: Tensor | None = None,
    cu_seqlens_k: Tensor | None = None,
    max_len_q: int | None = None,
    max_len_k: int | None = None,
    seqused_k: Tensor | None = None,
    scale: float | None = None,
    force_valu: bool = False,
    window: int | None = None,
    zero_padded_rows: bool = False,
) -> Tensor:
    """Multi-row attention (``asrattn_fwd``).  ``window`` (causal only):
    each query also skips keys more than ``window - 1`` before its last
    visible one (sliding-window attention).  ``zero_padded_rows`` (padded,
    non-causal, with ``seqused_k``): query rows at or past a sequence's key
    count are not computed and get zeros; the other rows are unchanged.

    Padded layout: ``q`` ``(batch, len_q, heads_q, head_dim)``, ``k``/``v``
    ``(batch, len_k, heads_kv, head_dim)``; packed layout (``cu_seqlens_*``
    given): ``(tokens, heads, head_dim)``.  Returns ``out`` in ``q``'s layout
    (a new contiguous tensor unless ``out`` is given).
    """
    flags = _lib.FWD_ZERO_PADDED_ROWS if zero_padded_rows else 0
    params, out, device, keep = _fwd_params(
        q, k, v, out, causal, cu_seqlens_q, cu_seqlens_k, max_len_q, max_len_k, seqused_k, scale, force_valu,
        window or 0, flags,
    )
    lib = _lib.load()
    _lib.check(lib.asrattn_fwd(ctypes.byref(params), _stream(device)), "asrattn_fwd")
    del keep
    return out


def flash_fsmn(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    weight: Tensor,
    *,
    seqused_k: Tensor | None = None,
    bias: Tensor | None = None,
    out: Tensor | None = None,
    memory: Tensor | None = None,
    scale: float | None = None,
    force_valu: bool = False,
    zero_padded_rows: bool = False,
) -> tuple[Tensor, Tensor]:
    """SAN-M self-attention and its FSMN memory in one call
    (``asrattn_fwd_fsmn``; ``sensevoice.py:97-135``).

    ``q``/``k``/``v`` ``(batch, frames, heads, head_dim)`` (views of the
    fused projection), ``seqused_k`` the int32 frame counts (or None: every
    frame is real), ``weight`` the depthwise Conv1d weight ``(C, 1, K)`` or
    ``(C, K)`` with ``C = heads * head_dim``.  Returns ``(out, memory)``,
    ``memory`` ``(batch, frames, C)`` = the reference's FSMN memory plus
    ``bias`` (if given) on every row.  ``zero_padded_rows`` (with
    ``seqused_k``): attention rows of frames at or past a sequence's count
    are zeros instead of computed; the memory is unaffected.
    """
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("the FSMN path needs q, k and v of one shape (batch, frames, heads, head_dim)")
    batch, frames, heads, head_dim = q.shape
    channels = heads * head_dim
    weight = weight.reshape(weight.shape[0], weight.shape[-1]) if weight.dim() == 3 else weight
    if weight.dim() != 2 or weight.shape[0] != channels:
        raise ValueError(f"weight must be ({channels}, 1, K) or ({channels}, K), got {tuple(weight.shape)}")
    weight = weight.contiguous()
    if bias is not None:
        if bias.shape != (channels,):
            raise ValueError(f"bias must be ({channels},), got {tuple(bias.shape)}")
        bias = bias.contiguous()
    _dtype_code(q, weight, *(() if bias is None else (bias,)))
    if memory is None:
        memory = torch.empty((batch, frames, channels), dtype=q.dtype, device=q.device)
    elif memory.shape != (batch, frames, channels) or memory.dtype != q.dtype or memory.stride(-1) != 1:
        raise ValueError("memory must be a (batch, frames, channels) tensor of q's dtype with unit channel stride")
    params, out, device, keep = _fwd_params(
        q, k, v, out, _lib.CAUSAL_NONE, None, None, None, None, seqused_k, scale, force_valu, 0,
        _lib.FWD_ZERO_PADDED_ROWS if zero_padded_rows else 0,
    )
    _check_device(q, weight, bias, memory)
    f = _lib.FsmnParams()
    f.weight, f.bias, f.memory = weight.data_ptr(), _ptr(bias), memory.data_ptr()
    f.m_batch_stride, f.m_token_stride = memory.stride(0), memory.stride(1)
    f.kernel_size = weight.shape[1]
    lib = _lib.load()
    _lib.check(
        lib.asrattn_fwd_fsmn(ctypes.byref(params), ctypes.byref(f), _stream(device)), "asrattn_fwd_fsmn"
    )
    del keep
    return out, memory


def _decode_params(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    out: Tensor,
    seqused_k: Tensor | None,
    positions: Tensor | None,
    num_splits: int,
    scale: float | None,
    window: int = 0,
) -> _lib.DecodeParams:
    params = _lib.DecodeParams()
    params.q, params.k, params.v, params.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    params.q_batch_stride, params.q_head_stride = q.stride(0), q.stride(1)
    params.k_batch_stride, params.k_token_stride, params.k_head_stride = k.stride(0), k.stride(1), k.stride(2)
    params.v_batch_stride, params.v_token_stride, params.v_head_stride = v.stride(0), v.stride(1), v.stride(2)
    params.o_batch_stride, params.o_head_stride = out.stride(0), out.stride(1)
    params.seqused_k = _ptr(seqused_k)
    params.positions = _ptr(positions)
    params.batch = q.shape[0]
    params.heads_q = q.shape[1]
    params.heads_kv = k.shape[2]
    params.head_dim = q.shape[2]
    params.max_len_k = k.shape[1]
    params.num_splits = num_splits
    params.dtype = _dtype_code(q, k, v)
    params.scale = 1.0 / math.sqrt(q.shape[2]) if scale is None else scale
    params.window = 0 if window is None else window
    return params


def decode(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    seqused_k: Tensor | None = None,
    positions: Tensor | None = None,
    num_splits: int = 0,
    scale: float | None = None,
    out: Tensor | None = None,
    workspace: Tensor | None = None,
    pages: PageTable | None = None,
    window: int | None = None,
) -> Tensor:
    """One query per sequence over a cache (``asrattn_decode``, or
    ``asrattn_decode_paged`` with ``pages``).  ``window``: only the last
    ``window`` of each row's keys (sliding-window attention).

    ``q`` ``(batch, heads_q, head_dim)``; ``k``/``v`` ``(batch, length,
    heads_kv, head_dim)``, any strides with a unit last one (pass
    ``cache.transpose(1, 2)`` for a ``(batch, heads, length, head_dim)``
    cache), or with ``pages`` the pools ``(num_pages, page_size, heads_kv,
    head_dim)``.  Sequence ``b`` uses keys ``0 .. n_b - 1`` with ``n_b =
    seqused_k[b]`` (int32), ``positions[b] + 1`` (int64) or ``length``.
    ``workspace``: the split partials' memory (see :func:`workspace`).
    Returns ``(batch, heads_q, head_dim)``.
    """
    if q.dim() != 3 or k.dim() != 4 or v.shape != k.shape:
        raise ValueError(
            f"decode expects q (B, Hq, D) and k/v (B, L, Hkv, D); got {tuple(q.shape)}, "
            f"{tuple(k.shape)}, {tuple(v.shape)}"
        )
    if (pages is None and k.shape[0] != q.shape[0]) or k.shape[3] != q.shape[2]:
        raise ValueError("q and k disagree on batch or head_dim")
    if q.shape[1] % k.shape[2]:
        raise ValueError(f"{q.shape[1]} query heads are not a multiple of {k.shape[2]} kv heads")
    _dtype_code(q, k, v)
    q = _aligned(q, (0, 1))
    k, v = (_aligned(t, (0, 1, 2)) for t in (k, v))
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must match q's shape and dtype, with a unit last stride")
    if seqused_k is not None:
        seqused_k = _int32(seqused_k, "seqused_k")
    if positions is not None:
        if positions.dtype != torch.int64:
            raise TypeError(f"positions must be int64, got {positions.dtype}")
        positions = positions.contiguous()
    for lengths in (seqused_k, positions):
        if lengths is not None and lengths.shape != (q.shape[0],):
            raise ValueError(f"key counts must have shape ({q.shape[0]},), got {tuple(lengths.shape)}")
    device = _check_device(q, k, v, out, seqused_k, positions, None if pages is None else pages.block_table)
    params = _decode_params(q, k, v, out, seqused_k, positions, num_splits, scale, window)
    pk = None
    if pages is not None:
        pk, params.max_len_k = _paged(pages, k, v, q.shape[0])
        params.k_batch_stride = params.v_batch_stride = 0
    lib = _lib.load()
    workspace = _split_workspace(lib.asrattn_decode_workspace_size(ctypes.byref(params)), workspace, device)
    size = 0 if workspace is None else workspace.numel()
    if pk is None:
        status = lib.asrattn_decode(ctypes.byref(params), _ptr(workspace), size, _stream(device))
        _lib.check(status, "asrattn_decode")
    else:
        status = lib.asrattn_decode_paged(
            ctypes.byref(params), None, ctypes.byref(pk), _ptr(workspace), size, _stream(device)
        )
        _lib.check(status, "asrattn_decode_paged")
    return out


def decode_append(
    q: Tensor,
    k_new: Tensor,
    v_new: Tensor,
    k: Tensor,
    v: Tensor,
    positions: Tensor,
    *,
    q_norm: Tensor | None = None,
    k_norm: Tensor | None = None,
    eps: float = 1e-6,
    cos: Tensor | None = None,
    sin: Tensor | None = None,
    num_splits: int = 0,
    scale: float | None = None,
    out: Tensor | None = None,
    workspace: Tensor | None = None,
    pages: PageTable | None = None,
    window: int | None = None,
    v_norm: bool = False,
) -> Tensor:
    """A decoder step with its prologue fused in (``asrattn_decode_append``;
    with ``pages``, ``k``/``v`` are page pools as for :func:`decode`):
    q ``(batch, heads_q, head_dim)`` and the step's key ``k_new`` ``(batch,
    heads_kv, head_dim)`` get the per-head RMSNorm (``q_norm``/``k_norm``
    weights ``(head_dim,)``, or neither) and the rotary embedding (``cos``/
    ``sin`` ``(batch, head_dim)`` at each row's position, or neither); the
    new key and ``v_new`` are written to the cache ``k``/``v`` ``(batch,
    length, heads_kv, head_dim)`` at ``positions`` (int64), and the query
    attends keys ``0 .. positions[b]``.  Replaces the step path of
    ``TextAttention._project`` and ``step`` (``qwen3_asr.py:366-372``,
    ``:409-432``) and Whisper's cache scatter (``whisper.py:224-228``).
    ``v_norm``: ``v_new`` also gets the RMS norm, without weights, before it
    is written and used (Gemma 4, ``gemma4.py:515``, ``:522-532``).
    Returns ``(batch, heads_q, head_dim)``."""
    if q.dim() != 3 or k.dim() != 4 or v.shape != k.shape:
        raise ValueError(
            f"decode_append expects q (B, Hq, D) and k/v (B, L, Hkv, D); got {tuple(q.shape)}, "
            f"{tuple(k.shape)}, {tuple(v.shape)}"
        )
    batch, heads_kv, head_dim = q.shape[0] if pages is not None else k.shape[0], k.shape[2], k.shape[3]
    if q.shape[0] != batch or q.shape[2] != head_dim or q.shape[1] % heads_kv:
        raise ValueError("q and k disagree on batch, head_dim or head grouping")
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        if t.shape != (batch, heads_kv, head_dim):
            raise ValueError(f"{name} must be ({batch}, {heads_kv}, {head_dim}), got {tuple(t.shape)}")
    if (q_norm is None) != (k_norm is None) or (cos is None) != (sin is None):
        raise ValueError("q_norm/k_norm and cos/sin come in pairs")
    if positions.dtype != torch.int64 or positions.shape != (batch,):
        raise ValueError(f"positions must be int64 ({batch},)")
    _dtype_code(q, k, v, k_new, v_new)
    extras = [t for t in (q_norm, k_norm, cos, sin) if t is not None]
    for t in extras:
        if t.dtype != q.dtype:
            raise TypeError("norm weights and rotary tables must have the cache's dtype")
    if q_norm is not None and (q_norm.shape != (head_dim,) or k_norm.shape != (head_dim,)):
        raise ValueError(f"norm weights must be ({head_dim},)")
    if cos is not None and (cos.shape != (batch, head_dim) or sin.shape != (batch, head_dim)):
        raise ValueError(f"cos/sin must be ({batch}, {head_dim})")
    q = _aligned(q, (0, 1))
    k_new, v_new = (_aligned(t, (0, 1)) for t in (k_new, v_new))
    if q_norm is not None:
        q_norm, k_norm = q_norm.contiguous(), k_norm.contiguous()
    if cos is not None:
        cos, sin = cos.contiguous(), sin.contiguous()
    if k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("the cache needs a unit last stride (it is written in place)")
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must match q's shape and dtype, with a unit last stride")
    positions = positions.contiguous()
    device = _check_device(q, k, v, out, positions, k_new, v_new, *extras,
                           None if pages is None else pages.block_table)
    params = _decode_params(q, k, v, out, None, positions, num_splits, scale, window)
    pk = None
    if pages is not None:
        pk, params.max_len_k = _paged(pages, k, v, batch)
        params.k_batch_stride = params.v_batch_stride = 0
    app = _lib.AppendParams()
    app.k_new, app.v_new = k_new.data_ptr(), v_new.data_ptr()
    app.kn_batch_stride, app.kn_head_stride = k_new.stride(0), k_new.stride(1)
    app.vn_batch_stride, app.vn_head_stride = v_new.stride(0), v_new.stride(1)
    app.q_norm = _ptr(q_norm)
    app.k_norm = _ptr(k_norm)
    app.eps = eps
    app.cos, app.sin = _ptr(cos), _ptr(sin)
    app.rope_batch_stride = 0 if cos is None else cos.stride(0)
    app.v_norm = 1 if v_norm else 0
    lib = _lib.load()
    workspace = _split_workspace(lib.asrattn_decode_workspace_size(ctypes.byref(params)), workspace, device)
    size = 0 if workspace is None else workspace.numel()
    if pk is None:
        status = lib.asrattn_decode_append(ctypes.byref(params), ctypes.byref(app), _ptr(workspace), size,
                                           _stream(device))
        _lib.check(status, "asrattn_decode_append")
    else:
        status = lib.asrattn_decode_paged(ctypes.byref(params), ctypes.byref(app), ctypes.byref(pk),
                                          _ptr(workspace), size, _stream(device))
        _lib.check(status, "asrattn_decode_paged")
    return out


def local_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    rel: Tensor,
    lengths: Tensor,
    *,
    chunk: int,
    past: int,
    future: int,
    softcap: float,
    invalid: float,
    out: Tensor | None = None,
) -> Tensor:
    """Blocked local attention with relative position scores
    (``asrattn_local``; Gemma 4's audio attention, ``gemma4.py:240-282``):
    float32 ``q``/``k``/``v`` ``(batch, tokens, heads, head_dim)`` (already
    scaled as the module scales them), ``rel`` ``(positions, heads,
    head_dim)`` the relative keys of distances ``past .. 0``, ``lengths``
    int32 valid tokens per sequence.  Returns float32 ``(batch, tokens,
    heads, head_dim)``."""
    for name, t in (("q", q), ("k", k), ("v", v), ("rel", rel)):
        if t.dtype != torch.float32:
            raise TypeError(f"local_attention computes in float32; {name} is {t.dtype}")
        if t.stride(-1) != 1:
            raise ValueError(f"{name} needs a unit last stride")
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k and v must share one (batch, tokens, heads, head_dim) shape")
    batch, tokens, heads, head_dim = q.shape
    if rel.dim() != 3 or rel.shape[1:] != (heads, head_dim):
        raise ValueError(f"rel must be (positions, {heads}, {head_dim}), got {tuple(rel.shape)}")
    lengths = _int32(lengths, "lengths")
    if lengths.shape != (batch,):
        raise ValueError(f"lengths must be ({batch},)")
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    elif out.shape != q.shape or out.dtype != torch.float32 or out.stride(-1) != 1:
        raise ValueError("out must be a float32 tensor of q's shape with a unit last stride")
    device = _check_device(q, k, v, rel, lengths, out)
    if device.type != "cuda":
        raise RuntimeError(f"attention kernels run on the GPU only; got tensors on {device}")
    params = _lib.LocalParams()
    params.q, params.k, params.v, params.rel, params.out = (t.data_ptr() for t in (q, k, v, rel, out))
    for prefix, t in (("q", q), ("k", k), ("v", v), ("o", out)):
        for axis, stride in zip(("batch", "token", "head"), t.stride()[:3]):
            setattr(params, f"{prefix}_{axis}_stride", stride)
    params.rel_position_stride, params.rel_head_stride = rel.stride(0), rel.stride(1)
    params.lengths = lengths.data_ptr()
    params.batch, params.tokens, params.heads, params.head_dim = batch, tokens, heads, head_dim
    params.chunk, params.past, params.future, params.rel_positions = chunk, past, future, rel.shape[0]
    params.softcap, params.invalid = softcap, invalid
    lib = _lib.load()
    _lib.check(lib.asrattn_local(ctypes.byref(params), _stream(device)), "asrattn_local")
    return out


def greedy_choice(logits: Tensor, suppress: Tensor | None = None, *,
                  workspace: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """Greedy next token per row of float32 ``logits`` ``(rows, vocab)`` and
    its log-probability, in one pass (``asrattn_choose``): the argmax (first
    index among equal maxima) after setting ``suppress``-ed entries (bool or
    uint8 ``(vocab,)``) to -inf, and ``log_softmax`` at it.  Replaces the
    greedy path of ``whisper.py:962-974`` and ``qwen3_asr.py:1200-1210``;
    ``logits`` is not modified.  Returns int64 tokens and float32
    log-probabilities ``(rows,)``.  Rows are split over several workgroups,
    their partials in ``workspace`` (see :func:`workspace`)."""
    if logits.dim() != 2 or logits.dtype != torch.float32:
        raise ValueError("greedy_choice takes float32 (rows, vocab) logits")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()  # e.g. the transposed product of Whisper's tied head
    rows, vocab = logits.shape
    if suppress is not None:
        if suppress.shape != (vocab,) or suppress.dtype not in (torch.bool, torch.uint8):
            raise ValueError(f"suppress must be a bool or uint8 ({vocab},) mask")
        suppress = suppress.contiguous().view(torch.uint8)
    device = _check_device(logits, suppress)
    if device.type != "cuda":
        raise RuntimeError("greedy_choice runs on the GPU only")
    token = torch.empty(rows, dtype=torch.int64, device=device)
    logprob = torch.empty(rows, dtype=torch.float32, device=device)
    lib = _lib.load()
    workspace = _split_workspace(lib.asrattn_choose_workspace_size(rows, vocab), workspace, device)
    size = 0 if workspace is None else workspace.numel()
    _lib.check(
        lib.asrattn_choose(logits.data_ptr(), rows, vocab, logits.stride(0), _ptr(suppress), token.data_ptr(),
                           logprob.data_ptr(), _ptr(workspace), size, _stream(device)),
        "asrattn_choose",
    )
    return token, logprob


def decode_supported(dtype: torch.dtype, head_dim: int, group: int) -> bool:
    """Whether the decode kernel takes this element type, head size and
    number of query heads per kv head (``decode_supported`` of the library:
    head_dim 64/128/256, and 512 in bfloat16; 1, 2, 4 or 8 heads)."""
    sizes = (64, 128, 256, 512) if dtype == torch.bfloat16 else (64, 128, 256)
    return dtype in _DTYPES and head_dim in sizes and group in (1, 2, 4, 8)


_scope = threading.local()


@contextlib.contextmanager
def workspace(buffer: Tensor):
    """Use ``buffer`` -- caller-owned uint8 device memory -- for the split
    partials of every :func:`decode`, :func:`decode_append` and
    :func:`greedy_choice` call of this thread inside the block that passes
    no ``workspace`` of its own.  Size it once, at the largest shape the
    block runs (:func:`decode_workspace_size`,
    :func:`choice_workspace_size`); a call that needs more raises.  Its
    address stays fixed, so graphs captured inside the block replay it.
    Calls that share one buffer must run in stream order.

    Without a buffer, each call that splits takes a temporary from torch's
    caching allocator (stream-ordered; inside graph capture, from the
    graph's pool)."""
    if buffer.dtype != torch.uint8 or buffer.dim() != 1 or not buffer.is_contiguous():
        raise ValueError("a workspace is a contiguous 1-D uint8 tensor")
    previous = getattr(_scope, "buffer", None)
    _scope.buffer = buffer
    try:
        yield buffer
    finally:
        _scope.buffer = previous


def _split_workspace(need: int, given: Tensor | None, device: torch.device) -> Tensor | None:
    """The workspace of a call that needs ``need`` bytes: ``given``, else the
    thread's :func:`workspace` buffer, else a temporary."""
    if need == 0 or need == ctypes.c_size_t(-1).value:
        return given  # no split (or invalid parameters: the call reports why)
    buffer = given if given is not None else getattr(_scope, "buffer", None)
    if buffer is None:
        return torch.empty(need, dtype=torch.uint8, device=device)
    if buffer.dtype != torch.uint8 or buffer.dim() != 1 or not buffer.is_contiguous():
        raise ValueError("a workspace is a contiguous 1-D uint8 tensor")
    if buffer.device != device:
        raise ValueError(f"the workspace is on {buffer.device}, the call on {device}")
    if buffer.numel() < need:
        raise ValueError(f"the call needs {need} workspace bytes, the workspace holds {buffer.numel()}")
    return buffer


def decode_workspace_size(batch: int, heads_q: int, heads_kv: int, head_dim: int, max_len_k: int,
                          dtype: torch.dtype = torch.bfloat16, num_splits: int = 0) -> int:
    """Bytes of split partials a :func:`decode` / :func:`decode_append` call
    of these sizes needs (``asrattn_decode_workspace_size``; 0 when it runs
    unsplit).  Raises for sizes the library does not take."""
    params = _lib.DecodeParams()
    params.batch, params.heads_q, params.heads_kv, params.head_dim = batch, heads_q, heads_kv, head_dim
    params.max_len_k, params.num_splits, params.scale = max_len_k, num_splits, 1.0
    params.dtype = _lib.BF16 if dtype == torch.bfloat16 else _lib.F32
    lib = _lib.load()
    need = lib.asrattn_decode_workspace_size(ctypes.byref(params))
    if need == ctypes.c_size_t(-1).value:
        raise ValueError(lib.asrattn_last_error().decode("utf-8", "replace"))
    return int(need)


def choice_workspace_size(rows: int, vocab: int) -> int:
    """Bytes of partials :func:`greedy_choice` over ``(rows, vocab)`` logits
    needs (``asrattn_choose_workspace_size``)."""
    return int(_lib.load().asrattn_choose_workspace_size(rows, vocab))


def sdpa(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    mask: KeyPrefix | Tensor | None = None,
    is_causal: bool = False,
    *,
    enable_gqa: bool = False,
    scale: float | None = None,
) -> Tensor:
    """``F.scaled_dot_product_attention(query, key, value, attn_mask=mask,
    is_causal=is_causal, enable_gqa=enable_gqa)`` for ``(batch, heads,
    length, head_dim)`` tensors, with ``mask`` a :class:`KeyPrefix` or a
    boolean prefix mask.  ``is_causal`` is top-left aligned, as in torch.

    Returns the output as ``(batch, length_q, heads, head_dim)`` -- the
    layout the callers reshape to ``(batch, length_q, width)`` next -- so no
    transpose copy is needed.
    """
    if query.dim() != 4 or key.dim() != 4 or value.shape != key.shape:
        raise ValueError("sdpa expects 4-d (batch, heads, length, head_dim) tensors")
    if query.shape[1] != key.shape[1] and not enable_gqa:
        raise ValueError("query and key head counts differ; pass enable_gqa=True")
    if isinstance(mask, Tensor):
        mask = KeyPrefix.from_mask(mask)
    q = query.transpose(1, 2)
    k = key.transpose(1, 2)
    v = value.transpose(1, 2)
    batch, len_q, heads, head_dim = q.shape
    if len_q == 1:
        # One query per row: the split-K decode kernel.  A causal single query
        # sees key 0 only (top-left alignment).
        out = torch.empty((batch, 1, heads, head_dim), dtype=q.dtype, device=q.device)
        if is_causal:
            k, v = k[:, :1], v[:, :1]
        decode(
            q[:, 0],
            k,
            v,
            seqused_k=None if mask is None else mask.lengths,
            positions=None if mask is None else mask.positions,
            scale=scale,
            out=out[:, 0],
        )
        return out
    seqused = None
    if mask is not None:
        seqused = mask.lengths
        if seqused is None:
            seqused = (mask.positions + 1).clamp(max=k.shape[1]).to(torch.int32)
    return flash(
        q,
        k,
        v,
        causal=_lib.CAUSAL_TOP_LEFT if is_causal else _lib.CAUSAL_NONE,
        seqused_k=seqused,
        scale=scale,
    )


def varlen_attn(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    cu_seq_q: Tensor,
    cu_seq_k: Tensor,
    max_q: int,
    max_k: int,
    *,
    window_size: tuple[int, int] = (-1, -1),
    enable_gqa: bool = False,
    seqused_k: Tensor | None = None,
    num_splits: int | None = None,
    scale: float | None = None,
) -> Tensor:
    """``torch.nn.attention.varlen.varlen_attn`` with the arguments the
    reference uses (``sensevoice.py:115-125``, ``qwen3_asr.py:156-166``,
    ``qwen3_asr.py:414-425``): packed ``(tokens, heads, head_dim)`` tensors,
    int32 cumulative sequence starts, ``window_size=(-1, 0)`` for causal
    (bottom-right aligned) and ``(-1, -1)`` for none.  ``num_splits`` is a
    tuning hint of the flash kernel and has no effect here.
    """
    del num_splits
    if window_size not in ((-1, -1), (-1, 0)):
        raise ValueError(f"window_size {window_size} is not supported (only (-1, -1) and (-1, 0))")
    if query.shape[1] != key.shape[1] and not enable_gqa:
        raise ValueError("query and key head counts differ; pass enable_gqa=True")
    return flash(
        query,
        key,
        value,
        causal=_lib.CAUSAL_BOTTOM_RIGHT if window_size == (-1, 0) else _lib.CAUSAL_NONE,
        cu_seqlens_q=cu_seq_q,
        cu_seqlens_k=cu_seq_k,
        max_len_q=max_q,
        max_len_k=max_k,
        seqused_k=seqused_k,
        scale=scale,
    )
