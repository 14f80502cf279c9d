"""Quantized GEMM callables registered under the ``hip`` backend.

The three registered entry points keep the reference's calling convention
(``dispatcher/dispatcher.py:285-294``: tensors positional, scalars keyword):

* ``fp8_gemm(A, B, scale_a=1.0, scale_b=1.0)``  -- ``gemm.fp8_gemm``
  (reference: triton/gemm/gemm_kernels.py:104-122).  A [M, K], B [K, N]
  (pass ``W.t()`` for a K-major weight W[N, K]); result ``(A @ B) * sa * sb``.
* ``fp4_gemm(A, B, fmt="mxfp4")`` -- ``gemm.fp4_gemm``, new name in the
  reference's ``<category>.<function>`` scheme (dispatcher/registry.py:6-8);
  semantics of cuda/gemm/fp4_gemm.cu:92-146 with MXFP4 / NVFP4 scales.
* ``bf16_gemm(A, B)`` -- ``gemm.bf16_gemm`` (reference:
  triton/gemm/gemm_kernels.py:46-65, registered at dispatcher/registry.py:134):
  ``C = A @ B`` of bf16 A [M, K], B [K, N], fp32 accumulation and, as in the
  reference, an fp32 result by default.
* ``lora_fused_gemm(X, W, loraA, loraB, scales)`` -- ``gemm.lora_fused_gemm``
  (reference: lora_fused_gemm_kernel, cuda/gemm/grouped_gemm.cu:106-140):
  ``Y = X @ W + sum_l scales[l] * X @ loraA[l] @ loraB[l]`` in fp32 from bf16
  operands.
* ``grouped_gemm(A, B, num_groups)`` -- ``gemm.grouped_gemm``
  (reference: triton/gemm/gemm_kernels.py:164-182).  An int third argument
  means fixed-size groups A [G, M, K], B [G, K, N]; a 1-D integer tensor of
  G+1 offsets means variable-size groups over concatenated rows A [T, K]
  (cuda/gemm/grouped_gemm.cu:26-32, :77-104).

High-precision inputs (bf16 / fp16 / fp32) are quantized on the GPU first
(the REST/CLI wire format cannot carry fp8 or packed fp4, dispatcher
schemas); pre-quantized inputs are accepted too (see each docstring).
Outputs are allocated here with ``torch.empty`` on ``A.device`` and owned by
the caller; inputs are never modified.  Work is enqueued on the current
stream without synchronising.  Every path goes through ``libdsl_gemm.so``;
there is no CPU or eager fallback.
"""
from __future__ import annotations

import numbers
import threading
import weakref
from collections import OrderedDict

import torch

from . import _native as N
from . import quant as Q

_HIGH = (torch.bfloat16, torch.float16, torch.float32)
_FP8 = torch.float8_e4m3fn


_OUT_NAMES = {"bfloat16": torch.bfloat16, "bf16": torch.bfloat16,
              "float32": torch.float32, "fp32": torch.float32, "float": torch.float32}


def _as_dtype(dtype) -> torch.dtype:
    """An output dtype given as a torch.dtype or by name ("float32", "fp32",
    "bfloat16", "bf16", optionally prefixed "torch."), as scalar params arrive
    over the REST / CLI wire (dispatcher.py:285-294 passes them unchanged)."""
    if isinstance(dtype, torch.dtype):
        return dtype
    if isinstance(dtype, str):
        name = dtype.strip().lower()
        name = name[6:] if name.startswith("torch.") else name
        if name in _OUT_NAMES:
            return _OUT_NAMES[name]
    raise ValueError(f"unsupported out_dtype {dtype!r}; use bfloat16 or float32")


def _out_code(dtype) -> int:
    dtype = _as_dtype(dtype)
    if dtype == torch.bfloat16:
        return N.OUT_BF16
    if dtype == torch.float32:
        return N.OUT_F32
    raise ValueError(f"unsupported out_dtype {dtype}; use torch.bfloat16 or torch.float32")


def _dev_scalar(v, device) -> torch.Tensor:
    """A 1-element float32 device tensor from a python number or tensor."""
    if isinstance(v, torch.Tensor):
        if v.numel() != 1:
            raise ValueError("expected a single scale value")
        return v.reshape(1).to(device=device, dtype=torch.float32)
    return torch.full((1,), float(v), dtype=torch.float32, device=device)


def _out_tensor(out, rows: int, cols: int, out_dtype, device) -> torch.Tensor:
    """The output matrix: a new [rows, cols] tensor of out_dtype, or the
    caller's `out`, which the kernels write through (ldc = out.stride(0)), so
    it must be exactly [rows, cols] with unit column stride, bf16 or fp32,
    on the operands' device."""
    if out is None:
        return torch.empty((rows, cols), dtype=_as_dtype(out_dtype), device=device)
    if not isinstance(out, torch.Tensor):
        raise TypeError("out must be a tensor")
    if out.dim() != 2 or tuple(out.shape) != (rows, cols):
        raise ValueError(f"out must be [{rows}, {cols}] (got {list(out.shape)})")
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"out must be bfloat16 or float32 (got {out.dtype})")
    if out.device != device:
        raise ValueError(f"out is on {out.device}, the operands on {device}")
    if rows > 0 and cols > 0 and (out.stride(1) != 1 or out.stride(0) < cols):
        raise ValueError("out needs unit column stride and a row stride >= its columns")
    return out


def _require_gpu(*ts):
    dev = ts[0].device
    for t in ts:
        if t.device.type != "cuda":
            raise ValueError(f"tensors must be on a GPU device (got {t.device})")
        if t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


def _k_major(b_kn: torch.Tensor) -> torch.Tensor:
    """[K, N] operand -> contiguous [N, K] (free when B is W.t())."""
    w = b_kn.t()
    return w if w.is_contiguous() else w.contiguous()


# K-major copies of weight operands passed in the reference's [.., K, N]
# layout, kept per source tensor (see _k_major_weight).
_WEIGHT_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()
_WEIGHT_CACHE_SLOTS = 4
_weight_lock = threading.Lock()


def clear_weight_cache() -> None:
    """Drop the K-major weight copies _k_major_weight keeps."""
    with _weight_lock:
        _WEIGHT_CACHE.clear()


def _k_major_weight(b: torch.Tensor) -> torch.Tensor:
    """A weight operand whose last two dims are [K, N] (the reference's
    layout, triton/gemm/gemm_kernels.py:104-108, :164-169) as contiguous
    [.., N, K].  Free when b is the transpose view of K-major storage
    (W.t(), W.transpose(1, 2)).  Otherwise the transposed copy is made once
    and kept while the source tensor is alive and unmodified -- keyed by its
    address and view geometry, checked against a weak reference to its
    storage's tensor and its version counter (which in-place writes bump) --
    so a weight held in the [K, N] layout is not transposed again on every
    call.  At most _WEIGHT_CACHE_SLOTS copies are kept (least recently used
    dropped first); clear_weight_cache() drops them."""
    w = b.transpose(-1, -2)
    if w.is_contiguous():
        return w
    base = b._base if b._base is not None else b
    key = (b.data_ptr(), tuple(b.shape), tuple(b.stride()), b.dtype, str(b.device))
    ver = b._version
    with _weight_lock:
        hit = _WEIGHT_CACHE.get(key)
        if hit is not None and hit[0]() is base and hit[1] == ver:
            _WEIGHT_CACHE.move_to_end(key)
            return hit[2]
    packed = w.contiguous()
    with _weight_lock:
        _WEIGHT_CACHE[key] = (weakref.ref(base), ver, packed)
        _WEIGHT_CACHE.move_to_end(key)
        while len(_WEIGHT_CACHE) > _WEIGHT_CACHE_SLOTS:
            _WEIGHT_CACHE.popitem(last=False)
    return packed


def _u8(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)



def _gemm_ws(op: int, m: int, n: int, k: int, device) -> torch.Tensor | None:
    nbytes = N.lib().dsl_gemm_workspace_bytes(op, m, n, k)
    return torch.empty(nbytes // 4, dtype=torch.float32, device=device) if nbytes else None


# ----------------------------------------------------------- packed level --

def _expand_groups(s: torch.Tensor, group_size: int, K: int, dim: int) -> torch.Tensor:
    """Scales of G-element K groups as scales of 128-element groups: the
    128-group j lies inside G-group j // (G/128), so repeating each scale
    G/128 times gives the same sum, sum_g (sum_{k in g} a*b) * sa * sb
    (cuda/gemm/fp8_gemm.cu:84-97), split into 128-element partials."""
    if group_size == 128:
        return s
    r = group_size // 128
    return s.repeat_interleave(r, dim=dim).narrow(dim, 0, -(-K // 128)).contiguous()


def _check_group_size(group_size) -> int:
    if isinstance(group_size, bool) or not isinstance(group_size, numbers.Integral) \
            or group_size < 128 or group_size % 128 != 0:
        raise ValueError(f"group_size must be a positive multiple of 128 (got {group_size!r}): "
                         "the FP8 MFMA sums 128 K per instruction, so scale groups are whole "
                         "multiples of 128")
    return int(group_size)


def fp8_gemm_packed(qa, qw, scale_a, scale_b, *, block: bool = False, group: bool = False,
                    out_dtype=torch.bfloat16, out=None):
    """GEMM on packed E4M3 codes.

    qa [M, K] and qw [N, K] are contiguous uint8 (or float8_e4m3fn) codes.
    Per-tensor (default): scale_a / scale_b are 1-element float32 device
    tensors.  Block-scaled (block=True): scale_a [M, ceil(K/128)] and
    scale_b [ceil(N/128), ceil(K/128)] float32.  Groupwise (group=True, the
    reference's fp8_gemm_groupwise layout with G = 128,
    cuda/gemm/fp8_gemm.cu:67-75): scale_a [M, ceil(K/128)] and scale_b
    [ceil(K/128), N], one weight scale per output column per group.
    """
    if block and group:
        raise ValueError("block and group scales are exclusive")
    dev = _require_gpu(qa, qw, scale_a, scale_b)
    qa, qw = N.vec_rows(_u8(qa)), N.vec_rows(_u8(qw))
    M, K = qa.shape
    Nn, K2 = qw.shape
    if K != K2:
        raise ValueError(f"K mismatch: A has {K}, W has {K2}")
    scale_a = scale_a.contiguous().float()
    scale_b = scale_b.contiguous().float()
    nkg = -(-K // 128)
    if block:
        if tuple(scale_a.shape) != (M, nkg) or tuple(scale_b.shape) != (-(-Nn // 128), nkg):
            raise ValueError("block scales must be [M, ceil(K/128)] and [ceil(N/128), ceil(K/128)]")
    if group:
        if tuple(scale_a.shape) != (M, nkg) or tuple(scale_b.shape) != (nkg, Nn):
            raise ValueError("groupwise scales must be [M, ceil(K/128)] and [ceil(K/128), N]")
    mode = N.SCALE_BLOCK128 if block else (N.SCALE_GROUP128 if group else N.SCALE_TENSOR)
    c = _out_tensor(out, M, Nn, out_dtype, dev)
    ws = _gemm_ws(N.OP_FP8, M, Nn, K, dev)
    with torch.cuda.device(dev):
        N.call("dsl_fp8_gemm", N.ptr(qa), N.ptr(qw), N.ptr(c), M, Nn, K, c.stride(0),
               _out_code(c.dtype), mode, N.ptr(scale_a), N.ptr(scale_b), N.ptr(ws),
               0 if ws is None else ws.numel() * 4, N.stream_of(dev))
    return c


def fp4_gemm_packed(qa, sa, qw, sw, *, fmt: str = "mxfp4", global_a=None, global_w=None,
                    out_dtype=torch.bfloat16, out=None):
    """GEMM on packed E2M1 codes: qa [M, K/2], qw [N, K/2] uint8 (low nibble =
    even K).  MXFP4: sa [M, K/32], sw [N, K/32] E8M0 bytes.  NVFP4: sa [M, K/16],
    sw [N, K/16] E4M3 bytes plus 1-element float32 global scales."""
    dev = _require_gpu(qa, qw, sa, sw)
    qa, qw = N.vec_rows(_u8(qa)), N.vec_rows(_u8(qw))
    sa, sw = _u8(sa).contiguous(), _u8(sw).contiguous()
    M, Kh = qa.shape
    Nn, Kh2 = qw.shape
    if Kh != Kh2:
        raise ValueError(f"K mismatch: A has {2 * Kh}, W has {2 * Kh2}")
    K = 2 * Kh
    if fmt == "mxfp4":
        code, blk = N.FMT_MXFP4, 32
    elif fmt == "nvfp4":
        code, blk = N.FMT_NVFP4, 16
        if global_a is None or global_w is None:
            raise ValueError("nvfp4 needs global_a and global_w")
    else:
        raise ValueError(f"unknown fp4 format {fmt!r} (expected 'mxfp4' or 'nvfp4')")
    if tuple(sa.shape) != (M, K // blk) or tuple(sw.shape) != (Nn, K // blk):
        raise ValueError(f"{fmt} scales must be [M, K/{blk}] and [N, K/{blk}]")
    ga = _dev_scalar(global_a, dev) if global_a is not None else None
    gw = _dev_scalar(global_w, dev) if global_w is not None else None
    c = _out_tensor(out, M, Nn, out_dtype, dev)
    ws = _gemm_ws(N.OP_FP4, M, Nn, K, dev)
    with torch.cuda.device(dev):
        N.call("dsl_fp4_gemm", N.ptr(qa), N.ptr(qw), N.ptr(c), M, Nn, K, c.stride(0),
               _out_code(c.dtype), code, N.ptr(sa), N.ptr(sw), N.ptr(ga), N.ptr(gw), N.ptr(ws),
               0 if ws is None else ws.numel() * 4, N.stream_of(dev))
    return c


def grouped_fp8_gemm_packed(qx, sx, qw, sw, offsets, *, out_dtype=torch.bfloat16, out=None):
    """Variable-size grouped GEMM on E4M3 codes.

    qx [T, K] rows sorted by group, qw [G, N, K], offsets int32 [G+1] on the
    device (offsets[0] = 0, offsets[G] = T, non-decreasing), sx [T] per-row
    scales, sw [G, N] per-channel scales.  Returns y [T, N].
    """
    dev = _require_gpu(qx, qw, sx, sw, offsets)
    qx, qw = N.vec_rows(_u8(qx)), N.vec_rows(_u8(qw))
    T, K = qx.shape
    G, Nn, K2 = qw.shape
    if K != K2:
        raise ValueError(f"K mismatch: X has {K}, W has {K2}")
    if offsets.dim() != 1 or offsets.numel() != G + 1:
        raise ValueError(f"offsets must be 1-D with {G + 1} entries")
    offsets = offsets.to(torch.int32).contiguous()
    sx = sx.reshape(-1).float().contiguous()
    sw = sw.reshape(G, Nn).float().contiguous()
    if sx.numel() != T:
        raise ValueError("scale_x must have one entry per row")
    y = _out_tensor(out, T, Nn, out_dtype, dev)
    with torch.cuda.device(dev):
        N.call("dsl_grouped_fp8_gemm", N.ptr(qx), N.ptr(qw), N.ptr(y), N.ptr(offsets), G, T, Nn,
               K, y.stride(0), _out_code(y.dtype), N.ptr(sx), N.ptr(sw), N.stream_of(dev))
    return y


# ------------------------------------------------------ registered callables --

def bf16_gemm(A: torch.Tensor, B: torch.Tensor, *, out_dtype: torch.dtype = torch.float32,
              out=None):
    """BF16 GEMM ``C = A @ B`` with fp32 accumulation (fp32 result by default).

    A [M, K] and B [K, N] must be bfloat16, as the reference asserts
    (triton/gemm/gemm_kernels.py:47); K % 8 == 0.  ``B = W.t()`` of a
    contiguous W [N, K] is read in place; any other layout of B (or a
    non-contiguous A) is first copied to K-major rows on the GPU.
    """
    if A.dim() != 2 or B.dim() != 2:
        raise ValueError("bf16_gemm expects A [M, K] and B [K, N]")
    if A.dtype != torch.bfloat16 or B.dtype != torch.bfloat16:
        raise TypeError(f"bf16_gemm: A and B must be bfloat16 (got {A.dtype}, {B.dtype})")
    M, K = A.shape
    K2, Nn = B.shape
    if K != K2:
        raise ValueError(f"K mismatch: A is [{M}, {K}], B is [{K2}, {Nn}]")
    dev = _require_gpu(A, B)
    a = N.vec_rows(A)
    w = N.vec_rows(_k_major_weight(B))
    c = _out_tensor(out, M, Nn, out_dtype, dev)
    ws = _gemm_ws(N.OP_BF16, M, Nn, K, dev)
    with torch.cuda.device(dev):
        N.call("dsl_bf16_gemm", N.ptr(a), N.ptr(w), N.ptr(c), M, Nn, K, c.stride(0),
               _out_code(c.dtype), N.ptr(ws), 0 if ws is None else ws.numel() * 4,
               N.stream_of(dev))
    return c


def lora_fused_gemm(X: torch.Tensor, W: torch.Tensor, loraA: torch.Tensor, loraB: torch.Tensor,
                    scales) -> torch.Tensor:
    """``Y = X @ W + sum_l scales[l] * (X @ loraA[l]) @ loraB[l]``, fp32.

    X [M, K], W [K, N] (``W = Wt.t()`` of a K-major Wt [N, K] is read in
    place), loraA [L, K, R], loraB [L, R, N], all bf16; scales: L numbers or
    a float tensor [L].  K % 8 == 0 and L * R % 8 == 0.
    """
    for t, nm in ((X, "X"), (W, "W"), (loraA, "loraA"), (loraB, "loraB")):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"lora_fused_gemm: {nm} must be bfloat16 (got {t.dtype})")
    if X.dim() != 2 or W.dim() != 2 or loraA.dim() != 3 or loraB.dim() != 3:
        raise ValueError("lora_fused_gemm expects X [M,K], W [K,N], loraA [L,K,R], loraB [L,R,N]")
    M, K = X.shape
    K2, Nn = W.shape
    L, K3, R = loraA.shape
    if K != K2 or K != K3 or tuple(loraB.shape) != (L, R, Nn):
        raise ValueError("lora_fused_gemm: shapes do not match")
    dev = _require_gpu(X, W, loraA, loraB)
    x = N.vec_rows(X)
    w = N.vec_rows(_k_major(W))                                     # [N, K]
    a_t = N.vec_rows(loraA.permute(0, 2, 1).reshape(L * R, K))      # row l*R + r = A_l[:, r]
    b_t = N.vec_rows(loraB.permute(2, 0, 1).reshape(Nn, L * R))     # col l*R + r = B_l[r, :]
    if isinstance(scales, torch.Tensor):
        s = scales.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    else:
        s = torch.tensor([float(v) for v in scales], dtype=torch.float32, device=dev)
    if s.numel() != L:
        raise ValueError(f"lora_fused_gemm: {L} scales expected")
    y = torch.empty((M, Nn), dtype=torch.float32, device=dev)
    nb = N.lib().dsl_lora_gemm_workspace_bytes(M, Nn, K, R, L)
    ws = torch.empty(max(nb, 256) // 4, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        N.call("dsl_lora_gemm", N.ptr(x), N.ptr(w), N.ptr(a_t), N.ptr(b_t), N.ptr(s), N.ptr(y), M, Nn,
               K, R, L, Nn, N.ptr(ws), ws.numel() * 4, N.stream_of(dev))
    return y


def fp8_gemm(A: torch.Tensor, B: torch.Tensor, scale_a=1.0, scale_b=1.0, *,
             granularity: str | None = None, group_size: int = 128,
             out_dtype: torch.dtype = torch.bfloat16):
    """FP8 E4M3 GEMM ``C = (A @ B) * scale_a * scale_b`` (bf16 by default).

    * A [M, K], B [K, N] in bf16/fp16/fp32: both are quantized on the GPU.
      granularity "tensor" (default): amax/448 per tensor; "block": 1x128
      activation groups and 128x128 weight blocks; "group": the reference's
      groupwise form (cuda/gemm/fp8_gemm.cu:67-99), 1 x group_size groups
      along K for A and, for B, one scale per output column per group.
      scale_a / scale_b stay extra multipliers, as in the reference.
    * A, B in float8_e4m3fn: scale_a / scale_b are the dequantization scales:
      numbers (per-tensor); tensors [M, ceil(K/128)] and
      [ceil(N/128), ceil(K/128)] (block-scaled); or the reference's groupwise
      layout, scale_a [M, ceil(K/G)] and scale_b [ceil(K/G), N] with G =
      group_size.  2-D scales are told apart by scale_b's shape, or named
      by granularity="block" / "group".  Block-scaled products
      scale_a[m, g] * scale_b[n // 128, g] must be normal fp32 numbers (the
      large-M kernels rescale by their ratios); the quantizers floor every
      scale at 1e-12, as the reference's do (cuda/gemm/fp8_gemm.cu:134).
    group_size must be a multiple of 128 (the FP8 MFMA sums 128 K at a time;
    a larger G is the same sum with its scale repeated over G/128 groups).
    ``out_dtype=torch.float32`` reproduces the reference's fp32 output.
    """
    if A.dim() != 2 or B.dim() != 2:
        raise ValueError("fp8_gemm expects A [M, K] and B [K, N]")
    M, K = A.shape
    K2, Nn = B.shape
    if K != K2:
        raise ValueError(f"K mismatch: A is [{M}, {K}], B is [{K2}, {Nn}]")
    if granularity not in (None, "tensor", "block", "group"):
        raise ValueError(f"granularity must be 'tensor', 'block' or 'group', got {granularity!r}")
    G = _check_group_size(group_size)
    if granularity == "block" and G != 128:
        raise ValueError("block scales are 128 x 128; group_size applies to granularity='group'")
    dev = _require_gpu(A, B)
    if A.dtype in _HIGH and B.dtype in _HIGH:
        gran = granularity or "tensor"
        if gran == "tensor":
            qa, sa = Q.quant_fp8_tensor(A)
            qw, sw = Q.quant_fp8_tensor(B.t())
        elif gran == "block":
            qa, sa = Q.quant_fp8_blocks(A, 1, 128)
            qw, sw = Q.quant_fp8_blocks(B.t(), 128, 128)
        else:
            qa, sa = Q.quant_fp8_blocks(A, 1, G)
            qw, sw_rows = Q.quant_fp8_blocks(B.t(), 1, G)      # [N, ceil(K/G)]
            sa = _expand_groups(sa, G, K, 1)
            sw = _expand_groups(sw_rows.t(), G, K, 0)           # [ceil(K/128), N]
        if not (isinstance(scale_a, numbers.Number) and isinstance(scale_b, numbers.Number)):
            raise ValueError("with high-precision inputs scale_a/scale_b must be numbers")
        if scale_a != 1.0:
            sa = sa * float(scale_a)
        if scale_b != 1.0:
            sw = sw * float(scale_b)
        return fp8_gemm_packed(qa, qw, sa, sw, block=gran == "block", group=gran == "group",
                               out_dtype=out_dtype)
    if A.dtype == _FP8 and B.dtype == _FP8:
        qw = _k_major_weight(B)
        if isinstance(scale_a, torch.Tensor) and scale_a.dim() == 2:
            if not (isinstance(scale_b, torch.Tensor) and scale_b.dim() == 2):
                raise ValueError("block-scaled / groupwise fp8 needs 2-D scale_a and scale_b")
            if granularity == "tensor":
                raise ValueError("granularity='tensor' needs scalar scales")
            nkg, nkG = -(-K // 128), -(-K // G)
            gran = granularity
            if gran is None:
                if G == 128 and tuple(scale_b.shape) == (-(-Nn // 128), nkg):
                    gran = "block"
                elif tuple(scale_b.shape) == (nkG, Nn):
                    gran = "group"
                else:
                    raise ValueError(
                        f"scale_b {tuple(scale_b.shape)} is neither a 128x128 block layout "
                        f"[{-(-Nn // 128)}, {nkg}] nor the groupwise layout [{nkG}, {Nn}]")
            sa, sb = scale_a.to(dev), scale_b.to(dev)
            if gran == "group":
                if tuple(sa.shape) != (M, nkG) or tuple(sb.shape) != (nkG, Nn):
                    raise ValueError(f"groupwise scales must be [M, ceil(K/G)] = [{M}, {nkG}] "
                                     f"and [ceil(K/G), N] = [{nkG}, {Nn}]")
                sa = _expand_groups(sa.float(), G, K, 1)
                sb = _expand_groups(sb.float(), G, K, 0)
            return fp8_gemm_packed(A, qw, sa, sb, block=gran == "block", group=gran == "group",
                                   out_dtype=out_dtype)
        if granularity in ("block", "group"):
            raise ValueError(f"granularity={granularity!r} needs 2-D scale tensors")
        return fp8_gemm_packed(A, qw, _dev_scalar(scale_a, dev), _dev_scalar(scale_b, dev),
                               out_dtype=out_dtype)
    raise TypeError(f"fp8_gemm: unsupported dtypes {A.dtype}, {B.dtype}")


def fp4_gemm(A: torch.Tensor, B: torch.Tensor, scale_a=None, scale_b=None, *,
             fmt: str = "mxfp4", global_a=None, global_b=None,
             out_dtype: torch.dtype = torch.bfloat16):
    """FP4 (E2M1) GEMM ``C = A @ B`` with MXFP4 or NVFP4 block scales.

    * A [M, K], B [K, N] in bf16/fp16/fp32: quantized on the GPU with ``fmt``.
    * Pre-packed: A uint8 [M, K/2] and B uint8 [K/2, N] (the ``.t()`` view of
      packed weights W [N, K/2]) with scale_a / scale_b bytes ([M, K/32] /
      [N, K/32] E8M0 for MXFP4, [M, K/16] / [N, K/16] E4M3 for NVFP4; uint8,
      float8_e8m0fnu or float8_e4m3fn) and, for NVFP4, global_a / global_b
      (numbers or 1-element tensors).
    The scale tensors are positional after B, so ``run_from_spec`` can pass a
    pre-quantized problem as four tensor specs (dispatcher.py:285-294), with
    ``fmt`` and the NVFP4 global scales as scalar params.
    """
    if A.dim() != 2 or B.dim() != 2:
        raise ValueError("fp4_gemm expects 2-D A and B")
    if fmt not in ("mxfp4", "nvfp4"):
        raise ValueError(f"unknown fp4 format {fmt!r} (expected 'mxfp4' or 'nvfp4')")
    _require_gpu(A, B)
    if A.dtype in _HIGH and B.dtype in _HIGH:
        M, K = A.shape
        K2, Nn = B.shape
        if K != K2:
            raise ValueError(f"K mismatch: A is [{M}, {K}], B is [{K2}, {Nn}]")
        if fmt == "mxfp4":
            qa, sa = Q.quant_mxfp4(A)
            qw, sw = Q.quant_mxfp4(B.t())
            return fp4_gemm_packed(qa, sa, qw, sw, fmt="mxfp4", out_dtype=out_dtype)
        qa, sa, ga = Q.quant_nvfp4(A)
        qw, sw, gw = Q.quant_nvfp4(B.t())
        return fp4_gemm_packed(qa, sa, qw, sw, fmt="nvfp4", global_a=ga, global_w=gw,
                               out_dtype=out_dtype)
    if A.dtype == torch.uint8 and B.dtype == torch.uint8:
        if not (isinstance(scale_a, torch.Tensor) and isinstance(scale_b, torch.Tensor)):
            raise ValueError("pre-packed fp4 inputs need scale_a and scale_b tensors")
        return fp4_gemm_packed(A, scale_a, _k_major_weight(B), scale_b, fmt=fmt, global_a=global_a,
                               global_w=global_b, out_dtype=out_dtype)
    raise TypeError(f"fp4_gemm: unsupported dtypes {A.dtype}, {B.dtype}")


def _grouped_problems(A: torch.Tensor, B: torch.Tensor, problems: torch.Tensor, out_dtype):
    """Variable-size grouped GEMM over GemmProblem descriptors, the
    reference's grouped_gemm_variable (cuda/gemm/grouped_gemm.cu:26-32,
    :77-104, :150-156): problems [G, 6] integers (M, N, K, A_offset,
    B_offset, C_offset), offsets in elements of the flat A, B and C buffers
    (:95-97 use them as element offsets); group g computes C_g [M][N] =
    A_g [M][K] @ B_g [K][N], all row-major.  A and B are bf16 / fp16 / fp32
    and are quantized to E4M3 like the other grouped forms (per-row
    activation, per-channel weight scales).  C is a new flat buffer of
    max(C_offset + M*N) elements (fp32 for fp32 inputs, else bf16, or
    out_dtype), zero where no group writes.

    The descriptors are read on the host (their sizes choose the launches):
    groups that share (N, K) run as one grouped FP8 GEMM over the device
    offset table, one launch per distinct (N, K); M = 0, N = 0 groups are
    skipped and K = 0 groups leave their C block at zero.  K % 16 == 0."""
    if problems.shape[-1] != 6 or problems.dtype not in (torch.int32, torch.int64):
        raise ValueError("problems must be an int tensor [G, 6]: M, N, K, A_offset, B_offset, C_offset")
    if A.dim() != 1 or B.dim() != 1:
        raise ValueError("with problem descriptors A and B are flat 1-D buffers")
    if A.dtype not in _HIGH or B.dtype not in _HIGH:
        raise TypeError(f"grouped_gemm problems: A and B must be bf16, fp16 or fp32 (got {A.dtype}, {B.dtype})")
    dev = _require_gpu(A, B)
    P = problems.to("cpu", torch.int64).tolist()
    if out_dtype is None:
        out_dtype = torch.float32 if A.dtype == torch.float32 else torch.bfloat16
    out_dtype = _as_dtype(out_dtype)
    c_len = 0
    buckets: dict = {}
    for g, (m, n, k, ao, bo, co) in enumerate(P):
        if min(m, n, k, ao, bo, co) < 0:
            raise ValueError(f"problem {g}: negative size or offset {P[g]}")
        if ao + m * k > A.numel() or bo + k * n > B.numel():
            raise ValueError(f"problem {g}: A / B range outside the buffers")
        if m and n:
            c_len = max(c_len, co + m * n)
            if k:
                if k % 16:
                    raise ValueError(f"problem {g}: K={k} must be a multiple of 16")
                buckets.setdefault((n, k), []).append(g)
    C = torch.zeros(c_len, dtype=out_dtype, device=dev)
    for (n, k), gs in buckets.items():
        xs = [A[P[g][3]:P[g][3] + P[g][0] * k].view(P[g][0], k) for g in gs]
        X = xs[0] if len(xs) == 1 else torch.cat(xs)
        Bs = torch.stack([B[P[g][4]:P[g][4] + k * n].view(k, n) for g in gs])     # [Gb, K, N]
        rows = torch.tensor([0] + [P[g][0] for g in gs], dtype=torch.int64).cumsum(0)
        offsets = rows.to(device=dev, dtype=torch.int32)
        Y = grouped_gemm(X, Bs, offsets, out_dtype=out_dtype)
        for i, g in enumerate(gs):
            m, co = P[g][0], P[g][5]
            C[co:co + m * n].view(m, n).copy_(Y[int(rows[i]):int(rows[i + 1])])
    return C


def grouped_gemm(A: torch.Tensor, B: torch.Tensor, num_groups, scale_a=None, scale_b=None, *,
                 out_dtype: torch.dtype | None = None):
    """Grouped FP8 GEMM (MoE experts / LoRA adapters), one W per group.

    * ``num_groups`` an int: fixed-size groups, A [G, M, K], B [G, K, N]
      -> C [G, M, N] (the reference's batched form).
    * ``num_groups`` a 1-D integer tensor of G+1 offsets: variable-size
      groups, A [T, K] with rows sorted by group, B [G, K, N] -> C [T, N];
      empty groups are allowed.
    * ``num_groups`` a 2-D integer tensor [G, 6] of GemmProblem descriptors
      (M, N, K, A_offset, B_offset, C_offset; cuda/gemm/grouped_gemm.cu:26-32):
      every group has its own M, N and K, over flat A, B and C buffers (see
      _grouped_problems).
    High-precision inputs are quantized to E4M3 with per-row activation and
    per-channel weight scales, so bf16 inputs give an FP8 product, not the
    reference's unquantized bf16 batched product (grouped_gemm_kernel,
    triton/gemm/gemm_kernels.py:125-182): expect FP8 rounding (about 3% of
    an entry's magnitude per product, ~1e-2 of max|C| over K), not bf16's.
    float8_e4m3fn inputs need scale_a [T] and scale_b [G, N]; an fp8 B
    [G, K, N] that is not the transpose view of K-major [G, N, K] storage is
    transposed once and the copy kept (_k_major_weight).  The output dtype
    defaults to A.dtype (bf16 for fp8 and fp16 inputs).  scale_a / scale_b
    are positional after the third argument, so a pre-quantized problem
    travels over ``run_from_spec`` as five tensor specs [X, B, offsets,
    scale_a, scale_b] (dispatcher.py:285-294).
    """
    if isinstance(num_groups, torch.Tensor) and num_groups.dim() == 2:
        return _grouped_problems(A, B, num_groups, out_dtype)
    if isinstance(num_groups, torch.Tensor):
        offsets = num_groups
        if A.dim() != 2 or B.dim() != 3:
            raise ValueError("variable-size grouped_gemm expects A [T, K] and B [G, K, N]")
        G = B.shape[0]
        if offsets.dim() != 1 or offsets.numel() != G + 1:
            raise ValueError(f"offsets must have num_groups+1 = {G + 1} entries")
        X = A
        fixed = None
    elif isinstance(num_groups, numbers.Integral):
        G = int(num_groups)
        if A.dim() != 3 or B.dim() != 3 or A.shape[0] != G or B.shape[0] != G:
            raise ValueError("fixed-size grouped_gemm expects A [G, M, K], B [G, K, N]")
        Mg = A.shape[1]
        X = A.reshape(G * Mg, A.shape[2])
        offsets = torch.arange(0, G * Mg + 1, Mg, dtype=torch.int32, device=A.device)
        fixed = Mg
    else:
        raise TypeError("num_groups must be an int or a 1-D tensor of group offsets")
    dev = _require_gpu(A, B, offsets)
    T, K = X.shape
    _, K2, Nn = B.shape
    if K != K2:
        raise ValueError(f"K mismatch: A has {K}, B has {K2}")
    if out_dtype is None:
        out_dtype = torch.float32 if A.dtype == torch.float32 else torch.bfloat16
    out_dtype = _as_dtype(out_dtype)
    if X.dtype in _HIGH and B.dtype in _HIGH:
        # W[g, n, k] rows (a view when B is the transpose of K-major [G, N, K]
        # storage, else a copy; the high-precision weight is quantized on
        # every call anyway)
        qx, sx = Q.quant_fp8_blocks(X, 1, K)
        qw, sw = Q.quant_fp8_blocks(B.transpose(1, 2).reshape(G * Nn, K), 1, K)
    elif X.dtype == _FP8 and B.dtype == _FP8:
        if scale_a is None or scale_b is None:
            raise ValueError("fp8 grouped_gemm needs scale_a [T] and scale_b [G, N]")
        qx, sx = X, scale_a.to(dev)
        qw, sw = _k_major_weight(B), scale_b.to(dev)    # [G, N, K]
    else:
        raise TypeError(f"grouped_gemm: unsupported dtypes {A.dtype}, {B.dtype}")
    y = grouped_fp8_gemm_packed(qx, sx, qw.reshape(G, Nn, K), sw.reshape(G, Nn), offsets,
                                out_dtype=out_dtype)
    if A.dtype == torch.float16:
        y = y.to(torch.float16)
    return y.reshape(G, fixed, Nn) if fixed is not None else y
