"""Torch-tensor wrappers over the C ABI (``include/ygg_moe.h``).

Every function takes CUDA (HIP) tensors, allocates its outputs with torch on
the same device, and enqueues the HIP kernels on the current torch stream.
There is no CPU path: CPU tensors are rejected.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _native as N
from ._native import check, lib, ptr, stream_handle

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1}
ACT_CODE = {"none": 0, "gelu": 1, "relu": 2, "sigmoid": 3}
WFORMAT_CODE = {"f32": 0, "bf16": 1, "int8": 2, "pauli": 3, "pauli_f32": 4, "int8_pauli": 5}
INT8_FORMATS = ("int8", "int8_pauli")
# activation row layouts of pauli_grouped_linear
X_LAYOUT = {"blade": 0, "pauli": 1}
Y_LAYOUT = {"pauli": 0, "blade": 1}


def _dev(*tensors):
    for t in tensors:
        if t is not None:
            if not t.is_cuda:
                raise ValueError("yggdrasil_amd ops run on the GPU only (got a CPU tensor)")
            if not t.is_contiguous():
                raise ValueError("tensors must be contiguous")
    return tensors[0].device


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; use float32 or bfloat16") from None


def _check_layer_args(x, k, E, F, logits=None, residual=None, router_weight=None, router_bias=None, b_up=None,
                      b_down=None):
    """Shapes and dtypes of a layer call's tensors, checked before their pointers reach the kernels."""
    if x.dim() != 3 or x.shape[2] != 8:
        raise ValueError(f"x must be (N, d, 8), got {tuple(x.shape)}")
    Nt, d = x.shape[0], x.shape[1]
    if not 1 <= k <= min(8, E):
        raise ValueError(f"top_k={k} must lie in [1, min(8, E={E})]")
    if logits is not None and (logits.dtype != torch.float32 or tuple(logits.shape) != (Nt, E)):
        raise ValueError(f"logits must be float32 ({Nt}, {E}), got {logits.dtype} {tuple(logits.shape)}")
    if logits is None and (router_weight is None or router_bias is None):
        raise ValueError("need logits or the router's weight and bias")
    if router_weight is not None and tuple(router_weight.shape) != (E, 4):
        raise ValueError(f"router_weight must be ({E}, 4), got {tuple(router_weight.shape)}")
    if router_bias is not None and tuple(router_bias.shape) != (E,):
        raise ValueError(f"router_bias must be ({E},), got {tuple(router_bias.shape)}")
    if residual is not None and (residual.dtype != x.dtype or tuple(residual.shape) != tuple(x.shape)):
        raise ValueError("residual must have x's shape and dtype")
    for name, b, want in (("b_up", b_up, (E, F, 8)), ("b_down", b_down, (E, d, 8))):
        if b is not None and (b.dtype != torch.float32 or tuple(b.shape) != want):
            raise ValueError(f"{name} must be a prepared float32 bias {want}, got {b.dtype} {tuple(b.shape)}")


# ---------------------------------------------------------------------------
# operator boundary
# ---------------------------------------------------------------------------


def geom_matmul_workspace_bytes(M: int, K: int, N: int) -> int:
    return int(lib().ygg_geom_matmul_f32_workspace_bytes(M, K, N))


def geom_matmul(a: torch.Tensor, b: torch.Tensor, *, workspace: torch.Tensor | None = None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """``out[m, n] = sum_k gp(a[m, k], b[k, n])`` (fp32, blade order).

    Drop-in for ``rune.ops.batched.geom_matmul`` (``rune/ops/batched.py:320-344``):
    one fp32 Pauli MFMA product with ``a`` as the weight.  ``workspace`` (uint8,
    at least :func:`geom_matmul_workspace_bytes`) and ``out`` may be given to reuse
    buffers across calls; otherwise they are allocated here.
    """
    dev = _dev(a, b)
    if a.dtype != torch.float32 or b.dtype != torch.float32:
        raise ValueError("geom_matmul is fp32")
    if a.dim() != 3 or b.dim() != 3 or a.shape[2] != 8 or b.shape[2] != 8 or a.shape[1] != b.shape[0]:
        raise ValueError(f"shapes {tuple(a.shape)} x {tuple(b.shape)} do not form (M,K,8) x (K,N,8)")
    a, b = a.contiguous(), b.contiguous()
    M, K, _ = a.shape
    Nn = b.shape[1]
    if out is None:
        out = torch.empty((M, Nn, 8), device=dev, dtype=torch.float32)
    elif out.dtype != torch.float32 or tuple(out.shape) != (M, Nn, 8) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous float32 ({M}, {Nn}, 8) tensor")
    need = geom_matmul_workspace_bytes(M, K, Nn)
    if workspace is None:
        workspace = torch.empty((max(need, 1),), device=dev, dtype=torch.uint8)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace of {workspace.numel() * workspace.element_size()} bytes, {need} needed")
    check(lib().ygg_geom_matmul_f32_ws(ptr(a), ptr(b), ptr(out), M, K, Nn, ptr(workspace),
                                       workspace.numel() * workspace.element_size(), stream_handle(dev)),
          "geom_matmul")
    return out


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------


@dataclass
class Routing:
    """Result of :func:`route` (all on the device)."""

    topk_idx: torch.Tensor  # (N, k) int32, slot 0 = most probable
    topk_w: torch.Tensor  # (N, k) fp32, renormalised
    counts: torch.Tensor  # (E,) int32
    offsets: torch.Tensor  # (E+1,) int32
    perm: torch.Tensor  # (N*k,) int32, token of each expert-grouped row
    slot_pos: torch.Tensor  # (N, k) int32, row of each slot

    @property
    def k(self) -> int:
        return self.topk_idx.shape[1]


def router_energy_logits(x: torch.Tensor, router_weight: torch.Tensor, router_bias: torch.Tensor,
                         return_energy: bool = False):
    """CliffordRouter logits from grade energies (``clifford_router.py:54-90``). x: (N, d, 8)."""
    dev = _dev(x, router_weight, router_bias)
    Nt, d = x.shape[0], x.shape[1]
    E = router_weight.shape[0]
    logits = torch.empty((Nt, E), device=dev, dtype=torch.float32)
    energy = torch.empty((Nt, 4), device=dev, dtype=torch.float32) if return_energy else None
    # named so the fp32 copies live until the launch has been queued
    rw, rb = router_weight.float().contiguous(), router_bias.float().contiguous()
    check(lib().ygg_router_energy_logits(ptr(x), _dtype_code(x), Nt, d, ptr(rw), ptr(rb), E, ptr(logits), ptr(energy),
                                         stream_handle(dev)), "router_energy_logits")
    return (logits, energy) if return_energy else logits


def router_head_logits(x: torch.Tensor, head_weight: torch.Tensor) -> torch.Tensor:
    """Scalar part of CliffordLinear(d -> E) (``hlm.py:109,141-145``). x: (N, d, 8); head_weight (E, d, 8)."""
    dev = _dev(x)
    if x.dim() != 3 or x.shape[2] != 8 or not x.is_contiguous():
        raise ValueError(f"router_head_logits: x must be contiguous (N, d, 8), got {tuple(x.shape)}")
    Nt, d = x.shape[0], x.shape[1]
    E = head_weight.shape[0]
    if tuple(head_weight.shape) != (E, d, 8):
        raise ValueError(f"router_head_logits: head_weight must be (E, {d}, 8)")
    hw = head_weight.float().contiguous()
    logits = torch.empty((Nt, E), device=dev, dtype=torch.float32)
    check(lib().ygg_router_head_logits(ptr(x), _dtype_code(x), Nt, d, ptr(hw), E, ptr(logits), stream_handle(dev)),
          "router_head_logits")
    return logits


def route(logits: torch.Tensor, k: int, out: Routing | None = None, workspace: torch.Tensor | None = None) -> Routing:
    """Softmax, top-k (lowest index wins ties) and the expert counting sort.

    ``out`` (a Routing of the right shapes) and ``workspace`` (at least
    ``ygg_route_workspace_bytes`` bytes) are reused when given: no allocation then.
    """
    dev = _dev(logits)
    if logits.dtype != torch.float32 or logits.dim() != 2:
        raise ValueError("logits must be (N, E) float32")
    Nt, E = logits.shape
    L = lib()
    ws_bytes = L.ygg_route_workspace_bytes(Nt, E, k)
    i32 = dict(device=dev, dtype=torch.int32)
    if out is not None:
        if tuple(out.topk_idx.shape) != (Nt, k) or out.counts.numel() != E:
            raise ValueError("out routing buffers do not match (N, E, k)")
        r = out
    else:
        r = Routing(
            topk_idx=torch.empty((Nt, k), **i32),
            topk_w=torch.empty((Nt, k), device=dev, dtype=torch.float32),
            counts=torch.empty((E,), **i32),
            offsets=torch.empty((E + 1,), **i32),
            perm=torch.empty((Nt * k,), **i32),
            slot_pos=torch.empty((Nt, k), **i32),
        )
    ws = workspace if workspace is not None and workspace.numel() >= ws_bytes else \
        torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    check(L.ygg_route(ptr(logits), Nt, E, k, ptr(r.topk_idx), ptr(r.topk_w), ptr(r.counts), ptr(r.offsets),
                      ptr(r.perm), ptr(r.slot_pos), ptr(ws), ws_bytes, stream_handle(dev)), "route")
    return r


def route_pauli_rows(logits: torch.Tensor, k: int, x: torch.Tensor, out: Routing | None = None,
                     x_pauli: torch.Tensor | None = None, workspace: torch.Tensor | None = None):
    """:func:`route` and, in the same launches, x (N, d, 8) -> its Pauli rows (bf16: the half-rows of
    :func:`pauli_rows_from_blade`; fp32: those of :func:`pauli_rows_from_blade_f32`) -- the first launches
    of the layer for the Pauli weight formats.  Returns ``(Routing, x_pauli)``; ``out``, ``x_pauli`` and
    ``workspace`` are reused when given."""
    dev = _dev(logits, x)
    if logits.dtype != torch.float32 or logits.dim() != 2:
        raise ValueError("logits must be (N, E) float32")
    Nt, E = logits.shape
    if x.dim() != 3 or x.shape[0] != Nt or x.shape[2] != 8:
        raise ValueError(f"x must be ({Nt}, d, 8), got {tuple(x.shape)}")
    d = x.shape[1]
    shape = (Nt, 2, d, 4) if x.dtype == torch.bfloat16 else (Nt, d, 2, 2, 2)
    if x_pauli is None:
        x_pauli = torch.empty(shape, device=dev, dtype=x.dtype)
    elif tuple(x_pauli.shape) != shape or x_pauli.dtype != x.dtype or not x_pauli.is_contiguous():
        raise ValueError(f"x_pauli must be a contiguous {x.dtype} {shape} tensor")
    L = lib()
    ws_bytes = L.ygg_route_workspace_bytes(Nt, E, k)
    r = out if out is not None else Routing(
        topk_idx=torch.empty((Nt, k), device=dev, dtype=torch.int32),
        topk_w=torch.empty((Nt, k), device=dev, dtype=torch.float32),
        counts=torch.empty((E,), device=dev, dtype=torch.int32),
        offsets=torch.empty((E + 1,), device=dev, dtype=torch.int32),
        perm=torch.empty((Nt * k,), device=dev, dtype=torch.int32),
        slot_pos=torch.empty((Nt, k), device=dev, dtype=torch.int32))
    if tuple(r.topk_idx.shape) != (Nt, k) or r.counts.numel() != E:
        raise ValueError("out routing buffers do not match (N, E, k)")
    ws = workspace if workspace is not None and workspace.numel() >= ws_bytes else \
        torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    check(L.ygg_route_pauli_rows(ptr(logits), Nt, E, k, ptr(x), _dtype_code(x), d, ptr(r.topk_idx), ptr(r.topk_w),
                                 ptr(r.counts), ptr(r.offsets), ptr(r.perm), ptr(r.slot_pos), ptr(x_pauli), ptr(ws),
                                 ws_bytes, stream_handle(dev)), "route_pauli_rows")
    return r, x_pauli


def route_energy(x: torch.Tensor, router_weight: torch.Tensor, router_bias: torch.Tensor, k: int) -> Routing:
    """CliffordRouter.forward (``clifford_router.py:54-104``) and the counting sort in one call.

    x: (N, d, 8); router_weight (E, 4), router_bias (E,).  Up to 1024 tokens the
    grade-energy logits are computed inside the routing kernel.
    """
    dev = _dev(x, router_weight, router_bias)
    if x.dim() != 3 or x.shape[2] != 8 or not x.is_contiguous():
        raise ValueError(f"route_energy: x must be contiguous (N, d, 8), got {tuple(x.shape)}")
    Nt, d = x.shape[0], x.shape[1]
    E = router_weight.shape[0]
    if tuple(router_weight.shape) != (E, 4) or tuple(router_bias.shape) != (E,):
        raise ValueError("route_energy: router_weight must be (E, 4) and router_bias (E,)")
    L = lib()
    ws_bytes = L.ygg_route_workspace_bytes(Nt, E, k)
    i32 = dict(device=dev, dtype=torch.int32)
    r = Routing(topk_idx=torch.empty((Nt, k), **i32), topk_w=torch.empty((Nt, k), device=dev, dtype=torch.float32),
                counts=torch.empty((E,), **i32), offsets=torch.empty((E + 1,), **i32),
                perm=torch.empty((Nt * k,), **i32), slot_pos=torch.empty((Nt, k), **i32))
    scratch = torch.empty((max(Nt * E, 1),), device=dev, dtype=torch.float32)
    ws = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    rw, rb = router_weight.float().contiguous(), router_bias.float().contiguous()
    check(L.ygg_route_energy(ptr(x), _dtype_code(x), Nt, d, ptr(rw), ptr(rb), E, k, ptr(r.topk_idx), ptr(r.topk_w),
                             ptr(r.counts), ptr(r.offsets), ptr(r.perm), ptr(r.slot_pos), ptr(scratch), ptr(ws),
                             ws_bytes, stream_handle(dev)), "route_energy")
    return r


def dispatch(x: torch.Tensor, routing: Routing, mask_order: bool = False,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """Expert-grouped copy of the token rows: ``out[slot_pos[t, s]] = x[t]``. x: (N, d, 8)."""
    dev = _dev(x)
    Nt, d = x.shape[0], x.shape[1]
    k = routing.k
    if out is None:
        out = torch.empty((Nt * k, d, 8), device=dev, dtype=x.dtype)
    elif tuple(out.shape) != (Nt * k, d, 8) or out.dtype != x.dtype:
        raise ValueError("out must be (N*k, d, 8) of x's dtype")
    check(lib().ygg_dispatch(ptr(x), _dtype_code(x), Nt, k, d, ptr(routing.slot_pos), ptr(out), int(mask_order),
                             stream_handle(dev)), "dispatch")
    return out


def combine(y_sorted: torch.Tensor, routing: Routing, residual: torch.Tensor | None = None,
            y_mask_order: bool = False, out_dtype: torch.dtype | None = None,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """Weighted combine in ascending expert order (+ residual). y_sorted: (N*k, d, 8)."""
    dev = _dev(y_sorted, residual)
    Nt, k = routing.topk_idx.shape
    d = y_sorted.shape[1]
    out_dtype = out_dtype or y_sorted.dtype
    if residual is not None and residual.dtype != out_dtype:
        raise ValueError("residual dtype must equal the output dtype")
    if out is None:
        out = torch.empty((Nt, d, 8), device=dev, dtype=out_dtype)
    elif tuple(out.shape) != (Nt, d, 8) or out.dtype != out_dtype:
        raise ValueError("out must be (N, d, 8) of the output dtype")
    check(lib().ygg_combine(ptr(y_sorted), _dtype_code(y_sorted), int(y_mask_order), Nt, k, d,
                            ptr(routing.topk_idx), ptr(routing.topk_w), ptr(routing.slot_pos), ptr(residual),
                            ptr(out), DTYPE_CODE[out_dtype], stream_handle(dev)), "combine")
    return out


# ---------------------------------------------------------------------------
# expert products
# ---------------------------------------------------------------------------


@dataclass
class PreparedWeights:
    """Expert weights in the device layout of one weight format."""

    data: torch.Tensor
    scales: torch.Tensor | None
    fmt: str
    E: int
    d_out: int
    d_in: int


def prepare_weights(w: torch.Tensor, fmt: str) -> PreparedWeights:
    """w: (E, d_out, d_in, 8) fp32 blade order -> prepared layout ('f32' | 'bf16' | 'int8' | 'pauli' |
    'pauli_f32' | 'int8_pauli').  The int8 formats also hold one fp32 scale per (expert, output channel):
    'int8' quantizes the blade components, 'int8_pauli' the entries of each weight's 2x2 complex matrix
    (the decode layer's format)."""
    dev = _dev(w)
    if w.dim() == 3:
        w = w.unsqueeze(0)
    w = w.float().contiguous()
    E, d_out, d_in, _ = w.shape
    code = WFORMAT_CODE[fmt]
    L = lib()
    nbytes = L.ygg_prepared_weight_bytes(E, d_out, d_in, code)
    if nbytes == 0:
        raise ValueError(f"weight format {fmt!r} cannot hold shape (E={E}, d_out={d_out}, d_in={d_in})")
    data = torch.empty((nbytes,), device=dev, dtype=torch.uint8)
    scales = torch.empty((E, d_out), device=dev, dtype=torch.float32) if fmt in INT8_FORMATS else None
    check(L.ygg_prepare_weights(ptr(w), E, d_out, d_in, code, ptr(data), ptr(scales), stream_handle(dev)),
          "prepare_weights")
    return PreparedWeights(data, scales, fmt, E, d_out, d_in)


def prepare_bias(b: torch.Tensor | None) -> torch.Tensor | None:
    """(E, d_out, 8) blade order -> mask order fp32."""
    if b is None:
        return None
    dev = _dev(b)
    b = b.float().contiguous()
    if b.dim() == 2:
        b = b.unsqueeze(0)
    E, d_out, _ = b.shape
    out = torch.empty_like(b)
    check(lib().ygg_prepare_bias(ptr(b), E, d_out, ptr(out), stream_handle(dev)), "prepare_bias")
    return out


def grouped_clifford_linear(x_sorted: torch.Tensor, pw: PreparedWeights, offsets: torch.Tensor,
                            bias_prepared: torch.Tensor | None = None, act: str = "none",
                            out_dtype: torch.dtype | None = None, out_blade_order: bool = True) -> torch.Tensor:
    """Per-expert CliffordLinear on expert-grouped rows. x_sorted: (P, d_in, 8) in mask order."""
    if pw.fmt in ("pauli", "pauli_f32", "int8_pauli"):
        raise ValueError("Pauli weights run through pauli_grouped_linear / pauli_grouped_linear_f32 / the decode "
                         "layer (int8_pauli)")
    dev = _dev(x_sorted, offsets, bias_prepared)
    P = x_sorted.shape[0]
    if x_sorted.shape[1] != pw.d_in:
        raise ValueError(f"x has d_in={x_sorted.shape[1]}, weights expect {pw.d_in}")
    want_x = torch.float32 if pw.fmt == "f32" else torch.bfloat16
    if x_sorted.dtype != want_x:
        raise ValueError(f"weight format {pw.fmt} takes {want_x} activations")
    out_dtype = out_dtype or x_sorted.dtype
    y = torch.empty((P, pw.d_out, 8), device=dev, dtype=out_dtype)
    check(lib().ygg_grouped_clifford_linear(ptr(x_sorted), P, ptr(pw.data), WFORMAT_CODE[pw.fmt], ptr(pw.scales),
                                            ptr(bias_prepared), ptr(offsets), pw.E, pw.d_in, pw.d_out,
                                            ACT_CODE[act], ptr(y), DTYPE_CODE[out_dtype], int(out_blade_order),
                                            stream_handle(dev)), "grouped_clifford_linear")
    return y


def pauli_grouped_linear(x: torch.Tensor, pw: PreparedWeights, offsets: torch.Tensor,
                         bias_prepared: torch.Tensor | None = None, act: str = "none", x_layout: str = "blade",
                         gather: torch.Tensor | None = None, rows: int | None = None, y_layout: str = "blade",
                         out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Per-expert CliffordLinear with Pauli (complex 2x2) weights.

    x_layout 'blade': x is (N, d_in, 8) bf16 in blade order; output row r reads
    x[gather[r]] (or x[r]).  x_layout 'pauli': x is (P, 2, d_in, 4) Pauli half-rows.
    y_layout 'pauli' returns (P, 2, d_out, 4) bf16; 'blade' returns (P, d_out, 8).
    ``rows`` is the number of product rows P (default: len(gather) or x's rows).
    """
    if pw.fmt != "pauli":
        raise ValueError("pauli_grouped_linear needs weights prepared with fmt='pauli'")
    dev = _dev(x, offsets, bias_prepared, gather)
    if x.dtype != torch.bfloat16:
        raise ValueError("Pauli products take bf16 activations")
    d_in_x = x.shape[1] if x_layout == "blade" else x.shape[2]
    if d_in_x != pw.d_in:
        raise ValueError(f"x has d_in={d_in_x}, weights expect {pw.d_in}")
    if rows is None:
        rows = gather.shape[0] if gather is not None else x.shape[0]
    if y_layout == "pauli":
        y = torch.empty((rows, 2, pw.d_out, 4), device=dev, dtype=torch.bfloat16)
    else:
        y = torch.empty((rows, pw.d_out, 8), device=dev, dtype=out_dtype)
    check(lib().ygg_pauli_grouped_linear(ptr(x), X_LAYOUT[x_layout], x.shape[0], ptr(gather), rows, ptr(pw.data),
                                         ptr(bias_prepared), ptr(offsets), pw.E, pw.d_in, pw.d_out, ACT_CODE[act],
                                         ptr(y), Y_LAYOUT[y_layout], DTYPE_CODE[y.dtype], stream_handle(dev)),
          "pauli_grouped_linear")
    return y


def pauli_grouped_linear_f32(x: torch.Tensor, pw: PreparedWeights, offsets: torch.Tensor,
                             bias_prepared: torch.Tensor | None = None, act: str = "none",
                             gather: torch.Tensor | None = None, rows: int | None = None,
                             y_layout: str = "blade") -> torch.Tensor:
    """fp32 per-expert CliffordLinear with Pauli weights (``fmt='pauli_f32'``).

    x: (rows, d_in, 2, 2, 2) fp32 Pauli rows (see :func:`pauli_rows_from_blade_f32`);
    output row r reads x[gather[r]] (or x[r]).  y_layout 'blade' -> (P, d_out, 8),
    'pauli' -> (P, d_out, 2, 2, 2).
    """
    if pw.fmt != "pauli_f32":
        raise ValueError("pauli_grouped_linear_f32 needs weights prepared with fmt='pauli_f32'")
    dev = _dev(x, offsets, bias_prepared, gather)
    if x.dtype != torch.float32 or x.dim() != 5 or tuple(x.shape[1:]) != (pw.d_in, 2, 2, 2):
        raise ValueError(f"x must be fp32 Pauli rows (rows, {pw.d_in}, 2, 2, 2)")
    if rows is None:
        rows = gather.shape[0] if gather is not None else x.shape[0]
    shape = (rows, pw.d_out, 2, 2, 2) if y_layout == "pauli" else (rows, pw.d_out, 8)
    y = torch.empty(shape, device=dev, dtype=torch.float32)
    check(lib().ygg_pauli_grouped_linear_f32(ptr(x), ptr(gather), rows, ptr(pw.data), ptr(bias_prepared),
                                             ptr(offsets), pw.E, pw.d_in, pw.d_out, ACT_CODE[act], ptr(y),
                                             Y_LAYOUT[y_layout], stream_handle(dev)), "pauli_grouped_linear_f32")
    return y


def pauli_rows_from_blade_f32(x: torch.Tensor) -> torch.Tensor:
    """(rows, d, 8) fp32 blade order -> (rows, d, 2, 2, 2) fp32 Pauli rows.

    Element [m, i, b, k, c] is the real (k = 0) or imaginary (k = 1) part of entry
    (c, b) of multivector x[m, i] as a 2x2 complex matrix.
    """
    dev = _dev(x)
    if x.dtype != torch.float32:
        raise ValueError("fp32 rows only")
    rows, d = x.shape[0], x.shape[1]
    out = torch.empty((rows, d, 2, 2, 2), device=dev, dtype=torch.float32)
    check(lib().ygg_pauli_rows_from_blade_f32(ptr(x), rows, d, ptr(out), stream_handle(dev)),
          "pauli_rows_from_blade_f32")
    return out


def pauli_rows_from_blade(x: torch.Tensor) -> torch.Tensor:
    """(rows, d, 8) bf16 blade order -> (rows, 2, d, 4) Pauli half-rows."""
    dev = _dev(x)
    if x.dtype != torch.bfloat16:
        raise ValueError("bf16 rows only")
    rows, d = x.shape[0], x.shape[1]
    out = torch.empty((rows, 2, d, 4), device=dev, dtype=torch.bfloat16)
    check(lib().ygg_pauli_rows_from_blade(ptr(x), rows, d, ptr(out), stream_handle(dev)), "pauli_rows_from_blade")
    return out


def grouped_experts(x_sorted: torch.Tensor, expert_offsets: torch.Tensor, expert_counts: torch.Tensor,
                    w_up: PreparedWeights, w_down: PreparedWeights, b_up: torch.Tensor | None = None,
                    b_down: torch.Tensor | None = None, act: str = "gelu", validate: bool = False) -> torch.Tensor:
    """Every expert's CliffordFFN on rows already grouped by expert: ``y_sorted``.

    The grouped-expert boundary of geoformer's ``FusedMoEExperts.forward(x_sorted,
    expert_offsets, expert_counts) -> y_sorted``
    (``geoformer/triton_kernels/fused_expert.py:306-331``), with this layer's expert
    (``CliffordFFN.forward``, ``holograph/models/hlm_block.py:55-61``: up product with
    bias and the grade-wise activation, then the down product with bias).

    x_sorted: (P, d, 8) blade order, or (P, 8 d) as geoformer passes it; the rows of
    expert e are ``expert_offsets[e] .. + expert_counts[e]``, the experts' ranges
    contiguous and ascending from row 0 (as a sort by expert leaves them).  Weights
    and biases are prepared (:func:`prepare_weights`, :func:`prepare_bias`); the
    weight format picks the products (bf16 / fp32 Pauli, or the L(w) blocks).
    ``validate`` checks the ranges on the host (one synchronisation).  Without it the
    ranges are clamped on the device (no synchronisation) into ascending bounds within
    ``[0, P]``, so malformed ranges give wrong rows, never accesses past x_sorted or y.
    Returns y_sorted in x_sorted's shape and dtype.
    """
    dev = _dev(x_sorted, expert_offsets, expert_counts, b_up, b_down)
    E, d, F = w_up.E, w_up.d_in, w_up.d_out
    if (w_down.E, w_down.d_in, w_down.d_out, w_down.fmt) != (E, F, d, w_up.fmt):
        raise ValueError("w_down must be (E, d, F) in w_up's format")
    flat = x_sorted.dim() == 2
    x = x_sorted.reshape(x_sorted.shape[0], d, 8) if flat else x_sorted
    if x.dim() != 3 or tuple(x.shape[1:]) != (d, 8):
        raise ValueError(f"x_sorted must be (P, {d}, 8) or (P, {8 * d}), got {tuple(x_sorted.shape)}")
    if expert_offsets.shape != (E,) or expert_counts.shape != (E,):
        raise ValueError(f"expert_offsets and expert_counts must have shape ({E},)")
    x = x.contiguous()
    P = x.shape[0]
    offs = torch.cat([expert_offsets.reshape(E), (expert_offsets[-1:] + expert_counts[-1:])]).to(torch.int32)
    if validate:
        o, c = expert_offsets.long().cpu(), expert_counts.long().cpu()
        if int(o[0]) != 0 or bool((c < 0).any()) or bool((o[1:] != o[:-1] + c[:-1]).any()) or int(o[-1] + c[-1]) != P:
            raise ValueError("expert ranges must be contiguous, ascending and cover the rows from 0")
    if P == 0:
        return x_sorted.clone()
    # the products take every range from these bounds: ascending and inside the rows
    offs = torch.cummax(offs.clamp(0, P), 0).values.to(torch.int32).contiguous()
    fmt = w_up.fmt
    if fmt == "int8_pauli":
        raise ValueError("int8_pauli weights run inside the decode layer (moe_forward), which routes its own "
                         "rows; use 'int8' for grouped experts")
    if fmt == "pauli":
        h = pauli_grouped_linear(x, w_up, offs, b_up, act, x_layout="blade", y_layout="pauli")
        y = pauli_grouped_linear(h, w_down, offs, b_down, "none", x_layout="pauli", y_layout="blade",
                                 out_dtype=x.dtype)
    elif fmt == "pauli_f32":
        h = pauli_grouped_linear_f32(pauli_rows_from_blade_f32(x), w_up, offs, b_up, act, y_layout="pauli")
        y = pauli_grouped_linear_f32(h, w_down, offs, b_down, "none", y_layout="blade")
    else:  # L(w) blocks read and write mask order between the products
        h = grouped_clifford_linear(to_mask_order(x), w_up, offs, b_up, act, out_blade_order=False)
        y = grouped_clifford_linear(h, w_down, offs, b_down, "none", out_dtype=x.dtype, out_blade_order=True)
    return y.reshape(x_sorted.shape) if flat else y


def moe_workspace_bytes(Nt: int, d: int, F: int, E: int, k: int, dtype: torch.dtype, fmt: str) -> int:
    return lib().ygg_moe_workspace_bytes(Nt, d, F, E, k, DTYPE_CODE[dtype], WFORMAT_CODE[fmt])


def moe_forward(x: torch.Tensor, k: int, w_up: PreparedWeights, w_down: PreparedWeights,
                b_up: torch.Tensor | None = None, b_down: torch.Tensor | None = None, act: str = "gelu",
                logits: torch.Tensor | None = None, router_weight: torch.Tensor | None = None,
                router_bias: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """The whole layer in one call (``ygg_moe_forward``). x: (N, d, 8). Returns (out, Routing-lite)."""
    dev = _dev(x, logits, residual, router_weight, router_bias, b_up, b_down)
    Nt, d = x.shape[0], x.shape[1]
    E, F = w_up.E, w_up.d_out
    if w_down.d_in != F or w_down.d_out != d or w_up.d_in != d or w_down.E != E:
        raise ValueError("expert weight shapes do not chain d -> F -> d")
    if w_up.fmt != w_down.fmt:
        raise ValueError("up and down weights must share a format")
    _check_layer_args(x, k, E, F, logits, residual, router_weight, router_bias, b_up, b_down)
    ws_bytes = moe_workspace_bytes(Nt, d, F, E, k, x.dtype, w_up.fmt)
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    if out is None:
        out = torch.empty_like(x)
    i32 = dict(device=dev, dtype=torch.int32)
    topk_idx = torch.empty((Nt, k), **i32)
    topk_w = torch.empty((Nt, k), device=dev, dtype=torch.float32)
    counts = torch.empty((E,), **i32)
    offsets = torch.empty((E + 1,), **i32)
    rw = router_weight.float().contiguous() if router_weight is not None else None
    rb = router_bias.float().contiguous() if router_bias is not None else None
    check(lib().ygg_moe_forward(ptr(x), _dtype_code(x), Nt, d, F, E, k, ACT_CODE[act], ptr(logits), ptr(rw),
                                ptr(rb), ptr(w_up.data), ptr(w_up.scales), ptr(b_up), ptr(w_down.data),
                                ptr(w_down.scales), ptr(b_down), WFORMAT_CODE[w_up.fmt], ptr(residual), ptr(out),
                                ptr(topk_idx), ptr(topk_w), ptr(counts), ptr(offsets), ptr(workspace), ws_bytes,
                                stream_handle(dev)), "moe_forward")
    return out, dict(topk_idx=topk_idx, topk_w=topk_w, counts=counts, offsets=offsets)


def clifford_layer_norm(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float = 1e-6,
                        out_dtype: torch.dtype | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """CliffordLayerNorm.forward (``normalization.py:44-67``). x: (..., d, 8); gamma, beta: (d, 8)."""
    dev = _dev(x, gamma, beta)
    if x.dim() < 2 or x.shape[-1] != 8 or not x.is_contiguous():
        raise ValueError(f"clifford_layer_norm: x must be contiguous (..., d, 8), got {tuple(x.shape)}")
    d = x.shape[-2]
    if tuple(gamma.shape) != (d, 8) or tuple(beta.shape) != (d, 8):
        raise ValueError(f"clifford_layer_norm: gamma and beta must be ({d}, 8)")
    Nt = x.numel() // (8 * d) if d else 0
    if out is None:
        out = torch.empty(x.shape, device=dev, dtype=out_dtype or x.dtype)
    elif tuple(out.shape) != tuple(x.shape) or not out.is_contiguous():
        raise ValueError("clifford_layer_norm: out must be a contiguous tensor of x's shape")
    g, b = gamma.float().contiguous(), beta.float().contiguous()
    check(lib().ygg_clifford_layer_norm(ptr(x), _dtype_code(x), Nt, d, ptr(g), ptr(b), float(eps), ptr(out),
                                        _dtype_code(out), stream_handle(dev)), "clifford_layer_norm")
    return out


def moe_block_ffn_workspace_bytes(Nt: int, d: int, F: int, E: int, k: int, dtype: torch.dtype, fmt: str) -> int:
    return lib().ygg_moe_block_ffn_workspace_bytes(Nt, d, F, E, k, DTYPE_CODE[dtype], WFORMAT_CODE[fmt])


def moe_block_ffn(x: torch.Tensor, k: int, norm_gamma: torch.Tensor, norm_beta: torch.Tensor, w_up: PreparedWeights,
                  w_down: PreparedWeights, b_up: torch.Tensor | None = None, b_down: torch.Tensor | None = None,
                  act: str = "gelu", logits: torch.Tensor | None = None, router_weight: torch.Tensor | None = None,
                  router_bias: torch.Tensor | None = None, norm_eps: float = 1e-6,
                  workspace: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """``x + moe(ffn_norm(x))`` in one call (``ygg_moe_block_ffn``, ``hlm_block.py:144-151``). x: (N, d, 8)."""
    dev = _dev(x, logits, norm_gamma, norm_beta, router_weight, router_bias, b_up, b_down)
    if x.dim() != 3 or x.shape[2] != 8 or not x.is_contiguous():
        raise ValueError(f"moe_block_ffn: x must be contiguous (N, d, 8), got {tuple(x.shape)}")
    Nt, d = x.shape[0], x.shape[1]
    E, F = w_up.E, w_up.d_out
    if w_down.d_in != F or w_down.d_out != d or w_up.d_in != d or w_down.E != E:
        raise ValueError("expert weight shapes do not chain d -> F -> d")
    if w_up.fmt != w_down.fmt:
        raise ValueError("up and down weights must share a format")
    _check_layer_args(x, k, E, F, logits, None, router_weight, router_bias, b_up, b_down)
    if tuple(norm_gamma.shape) != (d, 8) or tuple(norm_beta.shape) != (d, 8):
        raise ValueError(f"moe_block_ffn: norm gamma and beta must be ({d}, 8)")
    ws_bytes = moe_block_ffn_workspace_bytes(Nt, d, F, E, k, x.dtype, w_up.fmt)
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    if out is None:
        out = torch.empty_like(x)
    i32 = dict(device=dev, dtype=torch.int32)
    topk_idx = torch.empty((Nt, k), **i32)
    topk_w = torch.empty((Nt, k), device=dev, dtype=torch.float32)
    counts = torch.empty((E,), **i32)
    offsets = torch.empty((E + 1,), **i32)
    g, nb = norm_gamma.float().contiguous(), norm_beta.float().contiguous()
    rw = router_weight.float().contiguous() if router_weight is not None else None
    rb = router_bias.float().contiguous() if router_bias is not None else None
    check(lib().ygg_moe_block_ffn(ptr(x), _dtype_code(x), Nt, d, F, E, k, ACT_CODE[act], ptr(g), ptr(nb),
                                  float(norm_eps), ptr(logits), ptr(rw), ptr(rb), ptr(w_up.data), ptr(w_up.scales),
                                  ptr(b_up), ptr(w_down.data), ptr(w_down.scales), ptr(b_down),
                                  WFORMAT_CODE[w_up.fmt], ptr(out), ptr(topk_idx), ptr(topk_w), ptr(counts),
                                  ptr(offsets), ptr(workspace), ws_bytes, stream_handle(dev)), "moe_block_ffn")
    return out, dict(topk_idx=topk_idx, topk_w=topk_w, counts=counts, offsets=offsets)


# ---------------------------------------------------------------------------
# backward (fp32)
# ---------------------------------------------------------------------------


def adjoint_weights(w: torch.Tensor) -> torch.Tensor:
    """(E, d_out, d_in, 8) -> (E, d_in, d_out, 8): reverse of each weight, channel axes exchanged."""
    dev = _dev(w)
    if w.dtype != torch.float32 or w.dim() != 4 or w.shape[-1] != 8:
        raise ValueError("adjoint_weights: w must be fp32 (E, d_out, d_in, 8)")
    E, d_out, d_in = w.shape[:3]
    out = torch.empty((E, d_in, d_out, 8), device=dev, dtype=torch.float32)
    check(lib().ygg_adjoint_weights_f32(ptr(w), E, d_out, d_in, ptr(out), stream_handle(dev)), "adjoint_weights")
    return out


def grouped_weight_grad(dy: torch.Tensor, a: torch.Tensor, offsets: torch.Tensor, E: int,
                        gather: torch.Tensor | None = None, with_bias: bool = True):
    """dW[e, j, i] = sum over expert e's rows of dy[r, j] ~a[src(r), i]; (dW, db or None). fp32 blade order."""
    dev = _dev(dy, a, offsets, gather)
    d_out, d_in = dy.shape[1], a.shape[1]
    dW = torch.empty((E, d_out, d_in, 8), device=dev, dtype=torch.float32)
    db = torch.empty((E, d_out, 8), device=dev, dtype=torch.float32) if with_bias else None
    check(lib().ygg_grouped_weight_grad_f32(ptr(dy), ptr(a), ptr(gather), ptr(offsets), E, d_in, d_out, ptr(dW),
                                            ptr(db), stream_handle(dev)), "grouped_weight_grad")
    return dW, db


def grouped_weight_grad_pauli(dy_pauli: torch.Tensor, a_pauli: torch.Tensor, offsets: torch.Tensor, E: int,
                              gather: torch.Tensor | None = None, with_bias: bool = True,
                              workspace: torch.Tensor | None = None):
    """:func:`grouped_weight_grad` on the fp32 MFMA units from fp32 Pauli rows
    (:func:`pauli_rows_from_blade_f32`) of dy (P, d_out, 2, 2, 2) and a (.., d_in, 2, 2, 2)."""
    dev = _dev(dy_pauli, a_pauli, offsets, gather)
    for t in (dy_pauli, a_pauli):
        if t.dtype != torch.float32 or t.dim() != 5 or tuple(t.shape[2:]) != (2, 2, 2):
            raise ValueError("grouped_weight_grad_pauli: operands must be fp32 Pauli rows (rows, d, 2, 2, 2)")
    P, d_out, d_in = dy_pauli.shape[0], dy_pauli.shape[1], a_pauli.shape[1]
    dW = torch.empty((E, d_out, d_in, 8), device=dev, dtype=torch.float32)
    db = torch.empty((E, d_out, 8), device=dev, dtype=torch.float32) if with_bias else None
    ws_bytes = lib().ygg_grouped_weight_grad_pauli_f32_workspace_bytes(P, E, d_in, d_out)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    check(lib().ygg_grouped_weight_grad_pauli_f32(ptr(dy_pauli), ptr(a_pauli), ptr(gather), ptr(offsets), P, E, d_in,
                                                  d_out, ptr(dW), ptr(db), ptr(workspace), workspace.numel(),
                                                  stream_handle(dev)), "grouped_weight_grad_pauli")
    return dW, db


def activation_backward(h: torch.Tensor, grad_out: torch.Tensor, act: str) -> torch.Tensor:
    """Gradient w.r.t. the input of a grade-wise activation; h, grad_out (..., 8) fp32."""
    dev = _dev(h, grad_out)
    if h.shape != grad_out.shape or h.dtype != torch.float32 or grad_out.dtype != torch.float32:
        raise ValueError("activation_backward: h and grad_out must be fp32 tensors of one shape")
    out = torch.empty_like(h)
    check(lib().ygg_activation_backward(ptr(h), ptr(grad_out), h.numel() // 8, ACT_CODE[act], ptr(out),
                                        stream_handle(dev)), "activation_backward")
    return out


def moe_backward(x: torch.Tensor, k: int, w_up: PreparedWeights, w_up_adj: PreparedWeights, w_down: PreparedWeights,
                 w_down_adj: PreparedWeights, dout: torch.Tensor, b_up: torch.Tensor | None = None,
                 b_down: torch.Tensor | None = None, act: str = "gelu", logits: torch.Tensor | None = None,
                 router_weight: torch.Tensor | None = None, router_bias: torch.Tensor | None = None,
                 residual: bool = False, workspace: torch.Tensor | None = None, routing_grad: bool = True,
                 h_pre: torch.Tensor | None = None):
    """Backward of ``moe_forward`` (fp32, ``pauli_f32`` weights). Returns dx, dW_up, db_up, dW_down, db_down, dtopk_w.

    ``routing_grad=False`` skips the routing-weight gradient (dtopk_w is None), and with it
    the recompute of the expert outputs it needs.  ``h_pre``: the rows ``moe_forward_train``
    kept (then the up product is not recomputed).
    """
    dev = _dev(x, dout, logits)
    for pw in (w_up, w_up_adj, w_down, w_down_adj):
        if pw.fmt != "pauli_f32":
            raise ValueError("moe_backward: weights must be prepared as 'pauli_f32'")
    if x.dtype != torch.float32 or dout.dtype != torch.float32 or dout.shape != x.shape:
        raise ValueError("moe_backward: x and dout must be fp32 (N, d, 8) of one shape")
    Nt, d = x.shape[0], x.shape[1]
    E, F = w_up.E, w_up.d_out
    if (w_up_adj.d_out, w_up_adj.d_in, w_down.d_out, w_down.d_in, w_down_adj.d_out, w_down_adj.d_in) != \
            (d, F, d, F, F, d):
        raise ValueError("moe_backward: weight shapes do not chain d -> F -> d")
    _check_layer_args(x, k, E, F, logits, None, router_weight, router_bias, b_up, b_down)
    ws_bytes = lib().ygg_moe_backward_workspace_bytes(Nt, d, F, E, k)
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    f32 = dict(device=dev, dtype=torch.float32)
    dx = torch.empty_like(x)
    dWu, dbu = torch.empty((E, F, d, 8), **f32), torch.empty((E, F, 8), **f32)
    dWd, dbd = torch.empty((E, d, F, 8), **f32), torch.empty((E, d, 8), **f32)
    dtw = torch.empty((Nt, k), **f32) if routing_grad else None
    rw = router_weight.float().contiguous() if router_weight is not None else None
    rb = router_bias.float().contiguous() if router_bias is not None else None
    check(lib().ygg_moe_backward(ptr(x), Nt, d, F, E, k, ACT_CODE[act], ptr(logits), ptr(rw), ptr(rb),
                                 ptr(w_up.data), ptr(w_up_adj.data), ptr(b_up), ptr(w_down.data),
                                 ptr(w_down_adj.data), ptr(b_down), int(residual), ptr(dout), ptr(h_pre), ptr(dx),
                                 ptr(dWu),
                                 ptr(dbu), ptr(dWd), ptr(dbd), ptr(dtw), ptr(workspace), ws_bytes,
                                 stream_handle(dev)), "moe_backward")
    return dx, dWu, dbu, dWd, dbd, dtw


def moe_forward_train(x: torch.Tensor, k: int, w_up: PreparedWeights, w_down: PreparedWeights,
                      b_up: torch.Tensor | None = None, b_down: torch.Tensor | None = None, act: str = "gelu",
                      logits: torch.Tensor | None = None, router_weight: torch.Tensor | None = None,
                      router_bias: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                      workspace: torch.Tensor | None = None):
    """``moe_forward`` for a training step (fp32, ``pauli_f32``): also returns the up product's
    pre-activation rows ``h_pre`` (N k, F, 8) for ``moe_backward``."""
    dev = _dev(x, logits, residual, router_weight, router_bias, b_up, b_down)
    if w_up.fmt != "pauli_f32" or w_down.fmt != "pauli_f32" or x.dtype != torch.float32:
        raise ValueError("moe_forward_train: fp32 layers with 'pauli_f32' weights")
    Nt, d = x.shape[0], x.shape[1]
    E, F = w_up.E, w_up.d_out
    if w_down.d_in != F or w_down.d_out != d or w_up.d_in != d or w_down.E != E:
        raise ValueError("expert weight shapes do not chain d -> F -> d")
    _check_layer_args(x, k, E, F, logits, residual, router_weight, router_bias, b_up, b_down)
    ws_bytes = moe_workspace_bytes(Nt, d, F, E, k, x.dtype, w_up.fmt)
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    out = torch.empty_like(x)
    i32 = dict(device=dev, dtype=torch.int32)
    topk_idx, counts, offsets = torch.empty((Nt, k), **i32), torch.empty((E,), **i32), torch.empty((E + 1,), **i32)
    topk_w = torch.empty((Nt, k), device=dev, dtype=torch.float32)
    h_pre = torch.empty((Nt * k, F, 8), device=dev, dtype=torch.float32)
    rw = router_weight.float().contiguous() if router_weight is not None else None
    rb = router_bias.float().contiguous() if router_bias is not None else None
    check(lib().ygg_moe_forward_train(ptr(x), Nt, d, F, E, k, ACT_CODE[act], ptr(logits), ptr(rw), ptr(rb),
                                      ptr(w_up.data), ptr(b_up), ptr(w_down.data), ptr(b_down), ptr(residual),
                                      ptr(out), ptr(topk_idx), ptr(topk_w), ptr(counts), ptr(offsets), ptr(h_pre),
                                      ptr(workspace), ws_bytes, stream_handle(dev)), "moe_forward_train")
    return out, dict(topk_idx=topk_idx, topk_w=topk_w, counts=counts, offsets=offsets), h_pre


def grade_quantize(w: torch.Tensor, grade_bits=(8, 6, 6, 4), symmetric: bool = True, codes: bool = True):
    """Grade-aware quantization per leading index (``grade_quantize.py:153-238``).

    w: (T, ..., 8) fp32; each w[t] is one tensor with its own per-grade scale and
    zero point.  Returns ``(dequantized fp32 like w, codes int16 like w or None,
    scales (T, 4) float64, zero_points (T, 4) int32)``.
    """
    dev = _dev(w)
    if w.dtype != torch.float32 or w.dim() < 2 or w.shape[-1] != 8:
        raise ValueError("grade_quantize: w must be fp32 (T, ..., 8)")
    bits = [int(b) for b in grade_bits]
    if len(bits) != 4:
        raise ValueError("grade_quantize: need one bit width per grade (4)")
    T = w.shape[0]
    mv = w.numel() // (8 * T) if T else 0
    deq = torch.empty_like(w)
    cd = torch.empty(w.shape, device=dev, dtype=torch.int16) if codes else None
    sc = torch.empty((T, 4), device=dev, dtype=torch.float64)
    zp = torch.empty((T, 4), device=dev, dtype=torch.int32)
    host_bits = (ctypes.c_int32 * 4)(*bits)
    check(lib().ygg_grade_quantize(ptr(w), T, mv, ctypes.addressof(host_bits), int(symmetric), ptr(cd), ptr(sc),
                                   ptr(zp), ptr(deq), stream_handle(dev)), "grade_quantize")
    return deq, cd, sc, zp


def to_mask_order(x: torch.Tensor) -> torch.Tensor:
    """Blade order -> mask order (exchange components 3 and 4)."""
    return x[..., [0, 1, 2, 4, 3, 5, 6, 7]].contiguous()


def symbols() -> list[str]:
    return list(N.SIGNATURES)
