"""ctypes binding of ``libygg_moe.so`` (the gfx950 C-ABI library).

There is no CPU fallback: if the library is missing, or there is no GPU,
every operation raises.  ``torch`` is imported before the library is loaded
so that the library binds to the HIP runtime torch already loaded (both have
the soname ``libamdhip64.so.7``) -- one runtime, one device context.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede loading the library)

# YGG_MOE_LIB names another build of the same library (e.g. one with host-side sanitizers)
LIB_PATH = os.environ.get("YGG_MOE_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                                                         "libygg_moe.so")

_c_int, _c_size, _vp, _c_double = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_double

# symbol -> (restype, argtypes); must match include/ygg_moe.h
SIGNATURES = {
    "ygg_last_error": (ctypes.c_char_p, []),
    "ygg_version": (_c_int, []),
    "ygg_geom_matmul_f32": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "ygg_geom_matmul_f32_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "ygg_geom_matmul_f32_ws": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_size, _vp]),
    "ygg_router_head_logits": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _c_int, _vp, _vp]),
    "ygg_router_energy_logits": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp]),
    "ygg_route_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "ygg_route": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _vp]),
    "ygg_route_pauli_rows": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                      _vp, _vp, _c_size, _vp]),
    "ygg_route_energy": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _vp, _vp, _c_size, _vp]),
    "ygg_dispatch": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp]),
    "ygg_combine": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp]),
    "ygg_prepared_weight_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "ygg_prepare_weights": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "ygg_prepare_bias": (_c_int, [_vp, _c_int, _c_int, _vp, _vp]),
    "ygg_grouped_clifford_linear": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                                             _c_int, _vp, _c_int, _c_int, _vp]),
    "ygg_pauli_grouped_linear": (_c_int, [_vp, _c_int, _c_int, _vp, _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                                          _c_int, _vp, _c_int, _c_int, _vp]),
    "ygg_pauli_rows_from_blade": (_c_int, [_vp, _c_int, _c_int, _vp, _vp]),
    "ygg_pauli_grouped_linear_f32": (_c_int, [_vp, _vp, _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                              _c_int, _vp]),
    "ygg_pauli_rows_from_blade_f32": (_c_int, [_vp, _c_int, _c_int, _vp, _vp]),
    "ygg_moe_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ygg_moe_forward": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp,
                                 _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _c_size, _vp]),
    "ygg_moe_forward_noalloc": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp,
                                         _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ygg_adjoint_weights_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "ygg_grouped_weight_grad_f32": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "ygg_grouped_weight_grad_pauli_f32_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "ygg_grouped_weight_grad_pauli_f32": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp,
                                                   _c_size, _vp]),
    "ygg_activation_backward": (_c_int, [_vp, _vp, _c_size, _c_int, _vp, _vp]),
    "ygg_moe_backward_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "ygg_moe_backward": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _vp]),
    "ygg_moe_forward_train": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _vp]),
    "ygg_grade_quantize": (_c_int, [_vp, _c_int, _c_size, _vp, _c_int, _vp, _vp, _vp, _vp, _vp]),
    "ygg_clifford_layer_norm": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _c_double, _vp, _c_int, _vp]),
    "ygg_moe_block_ffn_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ygg_moe_block_ffn": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_double,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _c_size, _vp]),
}


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, failed to load, or reported an error."""


_lib = None


def lib():
    """Load (once) and return the typed library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryError(
                f"{LIB_PATH} is not built; run `python -m yggdrasil_amd.build` (there is no CPU fallback)")
        try:
            handle = ctypes.CDLL(LIB_PATH)
        except OSError as exc:  # pragma: no cover
            raise NativeLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = lib().ygg_last_error().decode(errors="replace")
        raise NativeLibraryError(f"{what}: {msg}" if what else msg)


def stream_handle(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
