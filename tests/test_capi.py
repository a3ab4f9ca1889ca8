"""CPU checks of the C-ABI library and of the host-side logic (no GPU calls).

* the library loads and exports exactly what ``include/ygg_moe.h`` declares,
  and the ctypes table in ``yggdrasil_amd/_native.py`` matches the header;
* pure host-side functions (sizes, argument validation) behave;
* the product path has no CPU fallback: CPU tensors are refused.
"""

import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "ygg_moe.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ygg_\w+)\s*\(", text)))


def test_header_matches_ctypes_table():
    from yggdrasil_amd import _native

    assert header_functions() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    lib = _native.lib()  # loads without touching a GPU
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (ygg_\w+)", out))
    assert exported == set(header_functions()), exported ^ set(header_functions())


def test_host_side_sizes():
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    assert L.ygg_version() == 1
    # route workspace: one histogram row per 32-token block (scanned in place), 256-byte aligned
    nb = (16384 + 31) // 32
    assert L.ygg_route_workspace_bytes(16384, 16, 2) == (nb * 16 * 4 + 255) // 256 * 256
    assert L.ygg_route_workspace_bytes(33, 5, 3) == 256
    # prepared weights: bf16 dual layout pads d_out to 32 and d_in to 2
    assert L.ygg_prepared_weight_bytes(32, 512, 128, 1) == 32 * 16 * 64 * 64 * 32
    assert L.ygg_prepared_weight_bytes(2, 5, 7, 1) == 2 * 1 * 4 * 64 * 32
    assert L.ygg_prepared_weight_bytes(2, 5, 7, 2) == 2 * 1 * 4 * 64 * 8
    assert L.ygg_prepared_weight_bytes(2, 5, 7, 0) == 2 * 5 * 7 * 32
    assert L.ygg_prepared_weight_bytes(2, 5, 7, 9) == 0
    # int8 Pauli: 8 channels x 32 inputs x 8 bytes per block, channels and inputs padded
    assert L.ygg_prepared_weight_bytes(32, 512, 128, 5) == 32 * 512 * 128 * 8
    assert L.ygg_prepared_weight_bytes(2, 5, 7, 5) == 2 * 1 * 1 * 2048
    assert L.ygg_prepared_weight_bytes(1, 9, 33, 5) == 2 * 2 * 2048


def test_argument_errors_are_reported_not_aborted():
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    # rejected before any launch: E > 64
    assert L.ygg_route(None, 10, 65, 2, None, None, None, None, None, None, None, 0, None) == -1
    assert b"E=65" in L.ygg_last_error()
    assert L.ygg_dispatch(None, 7, 1, 1, 1, None, None, 0, None) == -1
    assert b"dtype" in L.ygg_last_error()
    assert L.ygg_prepare_weights(None, 1, 1, 1, 5, None, None, None) == -1
    assert L.ygg_grouped_clifford_linear(None, 1, None, 2, None, None, None, 1, 1, 1, 1, None, 1, 0, None) == -1
    assert b"scales" in L.ygg_last_error()
    # Pauli products: odd d_in, unknown layouts, Pauli rows in fp32 are rejected before any launch
    assert L.ygg_pauli_grouped_linear(None, 0, 4, None, 4, None, None, None, 1, 3, 4, 0, None, 1, 1, None) == -1
    assert b"even" in L.ygg_last_error()
    assert L.ygg_pauli_grouped_linear(None, 5, 4, None, 4, None, None, None, 1, 2, 4, 0, None, 1, 1, None) == -1
    assert b"x layout" in L.ygg_last_error()
    assert L.ygg_pauli_grouped_linear(None, 1, 4, None, 4, None, None, None, 1, 2, 4, 0, None, 0, 0, None) == -1
    assert b"dtype" in L.ygg_last_error()
    # x of 2 GiB or more, gathered or not, is refused before any launch (32-bit staging offsets)
    big = (1 << 31) // (128 * 16) + 1
    assert L.ygg_pauli_grouped_linear(1, 1, big, 1, 64, 1, None, 1, 1, 128, 64, 0, 1, 1, 1, None) == -1
    assert b"2 GiB" in L.ygg_last_error()
    assert L.ygg_pauli_grouped_linear(1, 0, big, None, big, 1, None, 1, 1, 128, 64, 0, 1, 1, 1, None) == -1
    assert b"2 GiB" in L.ygg_last_error()
    # without a gather, x must hold every row the product reads
    assert L.ygg_pauli_grouped_linear(1, 1, 3, None, 4, 1, None, 1, 1, 8, 8, 0, 1, 1, 1, None) == -1
    assert b"without a gather" in L.ygg_last_error()
    assert L.ygg_prepared_weight_bytes(2, 4, 3, 3) == 0  # odd d_in has no Pauli layout
    assert L.ygg_prepared_weight_bytes(2, 4, 6, 3) == 2 * 4 * 6 * 16
    assert L.ygg_prepared_weight_bytes(2, 4, 3, 4) == 2 * 4 * 3 * 64  # fp32 Pauli takes odd d_in


def test_layer_rejects_bad_routing_sizes():
    """Every path of ygg_moe_forward checks E and k before any launch, including the int8
    decode path that routes inside its up product (k > E would leave slots unwritten)."""
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    ws = L.ygg_moe_workspace_bytes(8, 16, 32, 2, 2, 1, 2)

    def fwd(E, k, fmt=2, act=1):  # bf16 activations, int8 weights, given logits, dummy non-null pointers
        return L.ygg_moe_forward(1, 1, 8, 16, 32, E, k, act, 1, None, None, 1, 1, None, 1, 1, None, fmt, None, 1,
                                 1, 1, 1, 1, 1, ws, None)

    assert fwd(2, 3) == -1 and b"k=3" in L.ygg_last_error()
    assert fwd(2, 0) == -1 and b"k=0" in L.ygg_last_error()
    assert fwd(0, 1) == -1 and b"E=0" in L.ygg_last_error()
    assert fwd(65, 2) == -1 and b"E=65" in L.ygg_last_error()
    assert fwd(4, 9) == -1 and b"k=9" in L.ygg_last_error()
    assert fwd(2, 2, act=7) == -1 and b"activation" in L.ygg_last_error()
    # int8 weights without scales
    assert L.ygg_moe_forward(1, 1, 8, 16, 32, 2, 2, 1, 1, None, None, 1, None, None, 1, None, None, 2, None, 1,
                             1, 1, 1, 1, 1, ws, None) == -1
    assert b"scales" in L.ygg_last_error()
    # int8 Pauli weights: the one-launch decode layer takes at most 128 tokens and d <= 128
    for n_tok, dm in ((129, 16), (8, 129)):
        ws5 = L.ygg_moe_workspace_bytes(n_tok, dm, 32, 2, 2, 1, 5)
        assert L.ygg_moe_forward(1, 1, n_tok, dm, 32, 2, 2, 1, 1, None, None, 1, 1, None, 1, 1, None, 5, None, 1,
                                 1, 1, 1, 1, 1, ws5, None) == -1
        assert b"format 5" in L.ygg_last_error()
    assert fwd(2, 3, fmt=5) == -1 and b"k=3" in L.ygg_last_error()
    # fp32 activations cannot take int8 Pauli weights
    assert L.ygg_moe_forward(1, 0, 8, 16, 32, 2, 2, 1, 1, None, None, 1, 1, None, 1, 1, None, 5, None, 1,
                             1, 1, 1, 1, 1, ws, None) == -1
    assert b"does not match" in L.ygg_last_error()


def test_layer_refuses_unaddressable_sizes_before_any_launch():
    """The bf16 Pauli layer takes any number of tokens whose x fits the gathered rows' 2 GiB
    range (N = 73728 at the config 3 shape is accepted as far as the workspace check); beyond
    that, and beyond 2^31 - 1 token-expert rows, it refuses before the routing launches (dummy
    non-null pointers: nothing is dereferenced)."""
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()

    def fwd(N, d, F, E, k, ws_bytes):  # bf16, Pauli weights, given logits
        return L.ygg_moe_forward(1, 1, N, d, F, E, k, 1, 1, None, None, 1, None, None, 1, None, None, 3, None, 1,
                                 1, 1, 1, 1, 1, ws_bytes, None)

    # C3 shape beyond 32768 tokens: the sizes pass, the short workspace is what is refused
    assert fwd(73728, 128, 512, 32, 4, 0) == -1 and b"workspace" in L.ygg_last_error()
    assert L.ygg_moe_workspace_bytes(73728, 128, 512, 32, 4, 1, 3) > (1 << 31)
    # x's Pauli rows (N x 16 d bytes, gathered by token) past 2 GiB: refused with the reason
    assert fwd(1 << 20, 128, 512, 32, 2, 1 << 62) == -1
    assert b"gathered x rows" in L.ygg_last_error()
    # more token-expert rows than an int holds
    assert fwd(1 << 29, 8, 16, 16, 8, 1 << 62) == -1 and b"2^31 - 1" in L.ygg_last_error()
    # the block entry refuses the same sizes before its norm launches
    assert L.ygg_moe_block_ffn(1, 1, 1 << 20, 128, 512, 32, 2, 1, 1, 1, 1e-6, 1, None, None, 1, None, None, 1,
                               None, None, 3, 2, 1, 1, 1, 1, 1, 1 << 62, None) == -1
    assert b"gathered x rows" in L.ygg_last_error()


def test_backward_workspace_holds_either_weight_gradient():
    """The weight-gradient region is shared by the up (d -> F) and down (F -> d) products, so
    its size does not shrink below the down product's needs when d_model > d_ff."""
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    N, E, k, chunk = 1024, 4, 2, 384
    P = N * k
    chunks = (P + chunk - 1) // chunk + E

    def wg(d_in, d_out):  # per-chunk partial dW planes plus partial db planes, fp32
        return chunks * (d_out * d_in * 8 + d_out * 8) * 4

    def al(b):
        return (b + 255) // 256 * 256

    for d, F in ((32, 16), (16, 32)):
        regions = [N * k * 4, N * k * 4, E * 4, (E + 1) * 4, P * 4, P * 4, N * E * 4,
                   L.ygg_route_workspace_bytes(N, E, k), N * d * 32] + [P * F * 32] * 4 + [P * d * 32] * 3
        want = sum(al(r) for r in regions) + al(max(wg(d, F), wg(F, d)))
        assert L.ygg_moe_backward_workspace_bytes(N, d, F, E, k) == want, (d, F)


def test_config_validation():
    from yggdrasil_amd import MoEHLMConfig

    c = MoEHLMConfig(d_model=8, d_ff=16)
    assert c.weight_format == "pauli_f32"
    assert MoEHLMConfig(d_model=7, d_ff=5).weight_format == "pauli_f32"
    assert MoEHLMConfig(d_model=8, d_ff=16, weight_format="f32").weight_format == "f32"
    with pytest.raises(ValueError):
        MoEHLMConfig(d_model=8, d_ff=16, weight_format="pauli")
    with pytest.raises(ValueError):
        MoEHLMConfig(d_model=8, d_ff=16, dtype=torch.bfloat16, weight_format="pauli_f32")
    assert MoEHLMConfig(d_model=8, d_ff=16, dtype=torch.bfloat16).weight_format == "pauli"
    assert MoEHLMConfig(d_model=7, d_ff=16, dtype=torch.bfloat16).weight_format == "bf16"
    with pytest.raises(ValueError):
        MoEHLMConfig(d_model=7, d_ff=16, dtype=torch.bfloat16, weight_format="pauli")
    with pytest.raises(ValueError):
        MoEHLMConfig(d_model=8, d_ff=16, activation="swish")
    with pytest.raises(ValueError):
        MoEHLMConfig(d_model=8, d_ff=16, dtype=torch.float32, weight_format="int8")
    assert MoEHLMConfig(d_model=7, d_ff=5, dtype=torch.bfloat16, weight_format="int8_pauli").weight_format == \
        "int8_pauli"
    with pytest.raises(ValueError):  # fp32 layers, and d_model above the decode layer's 128
        MoEHLMConfig(d_model=8, d_ff=16, dtype=torch.float32, weight_format="int8_pauli")
    with pytest.raises(ValueError):
        MoEHLMConfig(d_model=256, d_ff=16, dtype=torch.bfloat16, weight_format="int8_pauli")
    with pytest.raises(ValueError):
        MoEHLMConfig(d_model=8, d_ff=16, n_experts=65)
    with pytest.raises(ValueError):
        MoEHLMConfig(d_model=8, d_ff=16, n_experts=4, top_k=5)


def test_no_cpu_fallback():
    from yggdrasil_amd import ops

    with pytest.raises(ValueError, match="GPU only"):
        ops.route(torch.zeros(4, 8), 2)
    with pytest.raises(ValueError, match="GPU only"):
        ops.geom_matmul(torch.zeros(2, 3, 8), torch.zeros(3, 4, 8))


def test_missing_library_raises(monkeypatch, tmp_path):
    from yggdrasil_amd import _native

    monkeypatch.setattr(_native, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_native, "_lib", None)
    with pytest.raises(_native.NativeLibraryError, match="no CPU fallback"):
        _native.lib()


def test_product_never_imports_oracle():
    pkg = os.path.join(ROOT, "yggdrasil_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", src, flags=re.M), f


def test_norm_and_block_argument_checks():
    """Rejections happen on the host, before any launch (no GPU needed)."""
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    assert L.ygg_clifford_layer_norm(None, 3, 4, 8, None, None, 1e-6, None, 0, None) == -1
    assert L.ygg_clifford_layer_norm(None, 0, 4, 0, None, None, 1e-6, None, 0, None) == -1
    assert L.ygg_clifford_layer_norm(None, 0, 4, 4097, None, None, 1e-6, None, 0, None) == -1
    assert L.ygg_clifford_layer_norm(None, 0, 4, 8, None, None, -1.0, None, 0, None) == -1
    assert L.ygg_clifford_layer_norm(None, 0, 4, 8, None, None, 1e-6, None, 0, None) == -1  # null pointers
    assert b"null" in L.ygg_last_error()
    assert L.ygg_clifford_layer_norm(None, 1, 0, 8, None, None, 1e-6, None, 1, None) == 0  # empty: nothing to do
    N, d, F, E, k = 300, 64, 256, 8, 2
    for dt, fmt, es in ((0, 4, 4), (1, 3, 2), (1, 2, 2)):
        moe = L.ygg_moe_workspace_bytes(N, d, F, E, k, dt, fmt)
        assert L.ygg_moe_block_ffn_workspace_bytes(N, d, F, E, k, dt, fmt) == (N * d * 8 * es + 255) // 256 * 256 + moe


def test_grade_quantize_argument_checks():
    import ctypes

    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    bits = (ctypes.c_int32 * 4)(8, 6, 6, 4)
    bad = (ctypes.c_int32 * 4)(8, 1, 6, 4)
    assert L.ygg_grade_quantize(None, 0, 0, ctypes.addressof(bits), 1, None, None, None, None, None) == 0
    assert L.ygg_grade_quantize(None, 2, 4, ctypes.addressof(bad), 1, None, None, None, None, None) == -1
    assert b"bit width" in L.ygg_last_error()
    assert L.ygg_grade_quantize(None, 2, 4, ctypes.addressof(bits), 1, None, None, None, None, None) == -1
    assert L.ygg_grade_quantize(None, 2, 4, None, 1, None, None, None, None, None) == -1


def test_weight_grad_pauli_argument_checks():
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    need = L.ygg_grouped_weight_grad_pauli_f32_workspace_bytes(3000, 4, 16, 32)
    # chunks of 384 rows: ceil(3000 / 384) + E partial planes of (d_out d_in + d_out) multivectors
    assert need == (8 + 4) * (32 * 16 * 8 + 32 * 8) * 4
    assert L.ygg_grouped_weight_grad_pauli_f32_workspace_bytes(-1, 4, 16, 32) == 0
    assert L.ygg_grouped_weight_grad_pauli_f32(None, None, None, None, 10, 2, 0, 4, None, None, None, 0, None) == -1
    assert b"bad sizes" in L.ygg_last_error()
    fake = 4096  # never dereferenced: the checks reject before any launch
    assert L.ygg_grouped_weight_grad_pauli_f32(fake, fake, None, fake, 3000, 4, 16, 32, fake, None, fake, need - 1,
                                               None) == -1
    assert b"workspace" in L.ygg_last_error()
    assert L.ygg_grouped_weight_grad_pauli_f32(None, None, None, fake, 10, 2, 4, 4, fake, None, fake, 1 << 20,
                                               None) == -1


def test_layer_wrappers_validate_tensors_before_launch():
    """ops' layer wrappers refuse logits, residuals, router parameters and biases of the wrong
    shape or dtype (host-side, before any pointer reaches a kernel)."""
    from yggdrasil_amd import ops

    N, d, F, E, k = 6, 4, 8, 3, 2
    x = torch.zeros(N, d, 8, dtype=torch.bfloat16)
    ok = dict(logits=torch.zeros(N, E), residual=torch.zeros(N, d, 8, dtype=torch.bfloat16),
              b_up=torch.zeros(E, F, 8), b_down=torch.zeros(E, d, 8))
    ops._check_layer_args(x, k, E, F, **ok)
    ops._check_layer_args(x, k, E, F, router_weight=torch.zeros(E, 4), router_bias=torch.zeros(E))
    bad = [
        dict(ok, logits=torch.zeros(N, E, dtype=torch.bfloat16)),
        dict(ok, logits=torch.zeros(N, E + 1)),
        dict(ok, residual=torch.zeros(N, d, 8)),
        dict(ok, residual=torch.zeros(N + 1, d, 8, dtype=torch.bfloat16)),
        dict(ok, b_up=torch.zeros(E, d, 8)),
        dict(ok, b_down=torch.zeros(E, d, 8, dtype=torch.bfloat16)),
        dict(logits=None),
        dict(logits=None, router_weight=torch.zeros(E, 3), router_bias=torch.zeros(E)),
        dict(logits=None, router_weight=torch.zeros(E, 4), router_bias=torch.zeros(E + 1)),
    ]
    for kw in bad:
        with pytest.raises(ValueError):
            ops._check_layer_args(x, k, E, F, **kw)
    for kk in (0, E + 1, 9):
        with pytest.raises(ValueError):
            ops._check_layer_args(x, kk, E, F, **ok)


def test_noalloc_entry_refuses_oversized_calls_before_touching_a_device():
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    limit = 64 << 20
    assert L.ygg_moe_workspace_bytes(8192, 128, 512, 32, 4, 1, 3) > limit
    rc = L.ygg_moe_forward_noalloc(1, 1, 8192, 128, 512, 32, 4, 1, 1, None, None, 1, None, None, 1, None, None, 3,
                                   None, 1, 1, 1, 1, 1, None)
    assert rc == -1 and b"more than the 67108864" in L.ygg_last_error()
    assert L.ygg_moe_forward_noalloc(1, 1, 8, 16, 32, 2, 0, 1, 1, None, None, 1, None, None, 1, None, None, 3,
                                     None, 1, 1, 1, 1, 1, None) == -1
    assert b"bad sizes" in L.ygg_last_error()
    # a decode-sized layer fits
    assert L.ygg_moe_workspace_bytes(64, 128, 512, 32, 2, 1, 2) <= limit


def test_geom_matmul_workspace_checks_before_touching_a_device():
    """The workspace form of the operator boundary sizes its scratch on the host and refuses a
    short workspace (or operands past 2^31 floats) with -1 and a message, before any launch."""
    from yggdrasil_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("library not built")
    L = _native.lib()
    M, K, N = 512, 128, 8192
    need = L.ygg_geom_matmul_f32_workspace_bytes(M, K, N)
    rnd = lambda b: (b + 255) // 256 * 256
    assert need == rnd(M * K * 64) + rnd(N * K * 32) + 256
    assert L.ygg_geom_matmul_f32_workspace_bytes(0, K, N) == 0
    fake = 1 << 20  # never dereferenced: every check below fails first
    assert L.ygg_geom_matmul_f32_ws(fake, fake, fake, M, K, N, fake, need - 1, None) == -1
    assert b"workspace" in L.ygg_last_error()
    assert L.ygg_geom_matmul_f32_ws(fake, fake, fake, M, K, N, None, need, None) == -1
    assert L.ygg_geom_matmul_f32_ws(fake, fake, fake, 4, 1 << 20, 1 << 10, fake, 1 << 40, None) == -1
    assert b"2^31" in L.ygg_last_error()
    assert L.ygg_geom_matmul_f32_ws(fake, fake, fake, -1, K, N, fake, need, None) == -1
    assert L.ygg_geom_matmul_f32_ws(None, fake, fake, M, K, N, fake, need, None) == -1
    # empty outputs are a no-op that touches nothing
    assert L.ygg_geom_matmul_f32_ws(None, None, None, 0, K, N, None, 0, None) == 0
