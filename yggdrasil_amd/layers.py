"""Drop-in torch modules for the MoE-HLM expert layer (host side, PyTorch-ROCm).

``CliffordMoELayer`` keeps the geoformer MoE module interface
``forward(x: (B, T, D)) -> (out: (B, T, D), aux_loss: 0-d tensor)``
(``geoformer/moe_hlm/router.py:97-142``, ``geoformer/triton_kernels/expert_gemm.py:192-254``)
with ``D = 8 d`` multivector-minor, and also accepts the holograph layout
``(B, T, d, 8)`` of ``HLMBlock._moe_forward`` (``holograph/models/hlm_block.py:154-183``),
whose arithmetic it computes: CliffordRouter gating (``holograph/layers/clifford_router.py:24-123``),
experts ``CliffordFFN`` = CliffordLinear -> grade-wise activation -> CliffordLinear
(``hlm_block.py:41-61``), and the weighted combine in ascending expert order.

All compute runs in the HIP library (``include/ygg_moe.h``); this module only
owns parameters, prepares the device weight layouts and allocates outputs.
There is no CPU path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import nn

from . import ops

ACTIVATIONS = ("gelu", "relu", "sigmoid")  # hlm_block.py:28-32
ROUTERS = ("energy", "logits", "clifford_head")


@dataclass
class MoEHLMConfig:
    """Layer configuration (mirrors HLMConfig's MoE fields, hlm_config.py:9-78).

    d_model     multivector channels d (flat width 8 d)
    d_ff        expert hidden width F (multivectors)
    n_experts   E (<= 64)
    top_k       k (<= 8)
    activation  'gelu' | 'relu' | 'sigmoid' (grade-wise)
    dtype       activation dtype: torch.float32 or torch.bfloat16
    weight_format  fp32 layers: 'pauli_f32' (the default: complex 2x2 weights on the fp32 MFMA
                units, 32 multiply-adds per multivector pair) or 'f32' (8x8 L(w) blocks on the
                vector units, 64); bf16 layers: 'pauli' (the default when d_model and d_ff are
                even), 'bf16' (8x8 L(w) blocks), 'int8' (per-output-channel int8, L(w) blocks) or
                'int8_pauli' (per-output-channel int8 of the complex 2x2 weights: the one-launch
                decode layer, batches of at most 128 tokens with d_model <= 128)
    router      'energy' -- CliffordRouter's grade-energy logits (default, the reference);
                'clifford_head' -- CliffordLinear(d -> E) then the scalar part;
                'logits' -- the caller passes logits to forward()
    """

    d_model: int
    d_ff: int
    n_experts: int = 4
    top_k: int = 2
    activation: str = "gelu"
    dtype: torch.dtype = torch.float32
    weight_format: str | None = None
    router: str = "energy"

    def __post_init__(self):
        if self.activation not in ACTIVATIONS:
            raise ValueError(f"activation must be one of {ACTIVATIONS}")
        if self.router not in ROUTERS:
            raise ValueError(f"router must be one of {ROUTERS}")
        if self.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("dtype must be float32 or bfloat16")
        even = self.d_model % 2 == 0 and self.d_ff % 2 == 0
        if self.weight_format is None:
            self.weight_format = "pauli_f32" if self.dtype == torch.float32 else ("pauli" if even else "bf16")
        if self.weight_format not in ("f32", "pauli_f32", "bf16", "int8", "pauli", "int8_pauli"):
            raise ValueError("weight_format must be 'f32', 'pauli_f32', 'bf16', 'int8', 'pauli' or 'int8_pauli'")
        if (self.dtype == torch.float32) != (self.weight_format in ("f32", "pauli_f32")):
            raise ValueError("fp32 layers use 'pauli_f32' or 'f32' weights; bf16 layers use 'pauli', 'bf16', "
                             "'int8' or 'int8_pauli'")
        if self.weight_format == "int8_pauli" and self.d_model > 128:
            raise ValueError("the 'int8_pauli' weight format serves d_model <= 128")
        if self.weight_format == "pauli" and not even:
            raise ValueError("the 'pauli' weight format needs even d_model and d_ff")
        if not 1 <= self.n_experts <= 64 or not 1 <= self.top_k <= min(8, self.n_experts):
            raise ValueError("need 1 <= n_experts <= 64 and 1 <= top_k <= min(8, n_experts)")


def xavier_clifford_init(d_out: int, d_in: int, generator=None) -> torch.Tensor:
    """Grade-wise Xavier init of a CliffordLinear weight (clifford_linear.py:58-81)."""
    w = torch.zeros(d_out, d_in, 8)
    fan = d_in + d_out
    for lo, hi in ((0, 1), (1, 4), (4, 7), (7, 8)):
        n = hi - lo
        w[..., lo:hi] = torch.randn(d_out, d_in, n, generator=generator) * math.sqrt(2.0 / (fan * n))
    return w


class CliffordMoELayer(nn.Module):
    """Routed mixture of CliffordFFN experts on Cl(3,0) multivectors."""

    def __init__(self, cfg: MoEHLMConfig, device=None, generator: torch.Generator | None = None):
        super().__init__()
        self.cfg = cfg
        E, d, F = cfg.n_experts, cfg.d_model, cfg.d_ff
        self.router_weight = nn.Parameter(torch.randn(E, 4, generator=generator) * 0.1)  # clifford_router.py:48
        self.router_bias = nn.Parameter(torch.zeros(E))  # clifford_router.py:49
        self.w_up = nn.Parameter(torch.stack([xavier_clifford_init(F, d, generator) for _ in range(E)]))
        self.b_up = nn.Parameter(torch.zeros(E, F, 8))
        self.w_down = nn.Parameter(torch.stack([xavier_clifford_init(d, F, generator) for _ in range(E)]))
        self.b_down = nn.Parameter(torch.zeros(E, d, 8))
        if cfg.router == "clifford_head":
            self.head_weight = nn.Parameter(xavier_clifford_init(E, d, generator))
        else:
            self.head_weight = None
        self._prepared = None
        self._workspace = None
        self.last_routing = None
        if device is not None:
            self.to(device)

    # -- parameters ----------------------------------------------------------
    @torch.no_grad()
    def load_reference_weights(self, router_weight=None, router_bias=None, w_up=None, b_up=None, w_down=None,
                               b_down=None, head_weight=None, grade_quant=None):
        """Copy weights given in the reference's layouts (blade order, fp32).

        ``grade_quant`` (a ``checkpoint.GradeQuantConfig``) passes each expert's
        up and down weight through grade-aware quantization on the GPU
        (``ygg_grade_quantize``, one scale per expert and grade, as the
        reference's mixed-precision layers) and keeps the dequantized values,
        which ``prepare()`` then lays out in the configured device format.
        """
        for name, val in (("router_weight", router_weight), ("router_bias", router_bias), ("w_up", w_up),
                          ("b_up", b_up), ("w_down", w_down), ("b_down", b_down), ("head_weight", head_weight)):
            if val is not None:
                p = getattr(self, name)
                p.copy_(torch.as_tensor(val, dtype=p.dtype, device=p.device).reshape(p.shape))
        if grade_quant is not None:
            if not self.w_up.is_cuda:
                raise ValueError("grade-aware quantization runs on the GPU: move the layer to the device first")
            for p in (self.w_up, self.w_down):
                deq, _, _, _ = ops.grade_quantize(p.detach().contiguous(), grade_quant.bits(), grade_quant.symmetric,
                                                  codes=False)
                p.copy_(deq)
        self._prepared = None

    def _param_versions(self):
        return tuple(p._version for p in self.parameters()) + (self.w_up.device,)

    @torch.no_grad()
    def prepare(self):
        """Build the device weight layouts (done lazily; redone when parameters change)."""
        fmt = self.cfg.weight_format
        head = None
        if self.head_weight is not None:
            head = self.head_weight.detach().float().contiguous()
        self._prepared = dict(
            key=self._param_versions(),
            w_up=ops.prepare_weights(self.w_up.detach(), fmt),
            w_down=ops.prepare_weights(self.w_down.detach(), fmt),
            b_up=ops.prepare_bias(self.b_up.detach()),
            b_down=ops.prepare_bias(self.b_down.detach()),
            head=head,
        )
        return self._prepared

    def _get_prepared(self):
        if self._prepared is None or self._prepared["key"] != self._param_versions():
            self.prepare()
        return self._prepared

    # -- forward ---------------------------------------------------------------
    def _head_logits(self, flat_x: torch.Tensor, prep) -> torch.Tensor:
        """CliffordLinear(d -> E) then grade 0 (hlm.py:109,141-145), bit-exact with the reference."""
        return ops.router_head_logits(flat_x, prep["head"])

    def moe_forward(self, x: torch.Tensor, logits: torch.Tensor | None = None,
                    residual: torch.Tensor | None = None) -> torch.Tensor:
        """``HLMBlock._moe_forward``: x (B, T, d, 8) -> (B, T, d, 8) (+ residual)."""
        cfg = self.cfg
        if x.dim() != 4 or x.shape[-1] != 8 or x.shape[-2] != cfg.d_model:
            raise ValueError(f"expected (B, T, {cfg.d_model}, 8), got {tuple(x.shape)}")
        if x.dtype != cfg.dtype:
            raise ValueError(f"layer dtype is {cfg.dtype}, input is {x.dtype}")
        B, T = x.shape[:2]
        flat = x.reshape(B * T, cfg.d_model, 8).contiguous()
        prep = self._get_prepared()
        if cfg.router == "logits":
            if logits is None:
                raise ValueError("router='logits' needs logits")
        elif cfg.router == "clifford_head" and logits is None:
            logits = self._head_logits(flat, prep)
        if logits is not None:
            logits = logits.reshape(B * T, cfg.n_experts).float().contiguous()
        res = residual.reshape(B * T, cfg.d_model, 8).contiguous() if residual is not None else None
        ws_bytes = ops.moe_workspace_bytes(B * T, cfg.d_model, cfg.d_ff, cfg.n_experts, cfg.top_k, cfg.dtype,
                                           cfg.weight_format)
        if self._workspace is None or self._workspace.numel() < ws_bytes or self._workspace.device != x.device:
            self._workspace = torch.empty((max(ws_bytes, 1),), device=x.device, dtype=torch.uint8)
        if self._needs_grad(x, residual):
            out = _MoEFunction.apply(flat, res, self.w_up, self.b_up, self.w_down, self.b_down, self, logits)
        else:
            out = self._forward_flat(flat, logits, res)
        return out.reshape(B, T, cfg.d_model, 8)

    def _forward_flat(self, flat, logits, res):
        cfg, prep = self.cfg, self._get_prepared()
        out, routing = ops.moe_forward(flat, cfg.top_k, prep["w_up"], prep["w_down"], prep["b_up"], prep["b_down"],
                                       cfg.activation, logits=logits,
                                       router_weight=self.router_weight.detach() if logits is None else None,
                                       router_bias=self.router_bias.detach() if logits is None else None,
                                       residual=res, workspace=self._workspace)
        self.last_routing = routing
        return out

    def _needs_grad(self, x, residual) -> bool:
        """Autograd runs for fp32 layers with 'pauli_f32' weights (the backward's format);
        other formats compute the forward only and their output carries no graph."""
        if not torch.is_grad_enabled() or self.cfg.weight_format != "pauli_f32":
            return False
        return x.requires_grad or (residual is not None and residual.requires_grad) or any(
            p.requires_grad for p in (self.w_up, self.b_up, self.w_down, self.b_down))

    @torch.no_grad()
    def _get_adjoint(self):
        """Adjoint expert weights (reverse, channel axes exchanged) in the 'pauli_f32' layout."""
        key = self._param_versions()
        if getattr(self, "_adjoint", None) is None or self._adjoint["key"] != key:
            self._adjoint = dict(key=key,
                                 w_up=ops.prepare_weights(ops.adjoint_weights(self.w_up.detach().contiguous()),
                                                          "pauli_f32"),
                                 w_down=ops.prepare_weights(ops.adjoint_weights(self.w_down.detach().contiguous()),
                                                            "pauli_f32"))
        return self._adjoint

    def forward(self, x: torch.Tensor, logits: torch.Tensor | None = None):
        """geoformer interface: (B, T, 8 d) or (B, T, d, 8) -> (same shape, aux_loss)."""
        flat_in = x.dim() == 3
        if flat_in:
            B, T, D = x.shape
            if D != 8 * self.cfg.d_model:
                raise ValueError(f"expected D = 8 * {self.cfg.d_model}, got {D}")
            x4 = x.reshape(B, T, self.cfg.d_model, 8)
        else:
            x4 = x
        out = self.moe_forward(x4, logits=logits)
        return (out.reshape(x.shape) if flat_in else out), self.aux_loss()

    def experts(self, x_sorted: torch.Tensor, expert_offsets: torch.Tensor,
                expert_counts: torch.Tensor) -> torch.Tensor:
        """geoformer's grouped-expert interface (``FusedMoEExperts.forward``,
        ``geoformer/triton_kernels/fused_expert.py:306-331``) over this layer's
        experts: rows already sorted by expert -> y_sorted (forward only)."""
        prep = self._get_prepared()
        return ops.grouped_experts(x_sorted, expert_offsets, expert_counts, prep["w_up"], prep["w_down"],
                                   prep["b_up"], prep["b_down"], self.cfg.activation)

    def aux_loss(self) -> torch.Tensor:
        """CliffordRouter.load_balance_loss (clifford_router.py:108-117) on this call's counts.

        The reference's formula sum_e (f_e - 1/E)^2 with f = counts / sum(counts); the
        reference never updates its counts and so always returns 0, this layer uses the
        counts of the last forward.
        """
        if self.last_routing is None:
            return torch.zeros((), device=self.w_up.device)
        c = self.last_routing["counts"].float()
        f = c / (c.sum() + 1e-12)
        return ((f - 1.0 / self.cfg.n_experts) ** 2).sum()


class _MoEFunction(torch.autograd.Function):
    """The layer as one autograd node: forward ``ygg_moe_forward``, backward ``ygg_moe_backward``.

    Gradients reach x, the residual and the expert weights and biases.  The
    routing is a constant of the backward, as in the reference, whose router
    has no backward (``hlm_block.py:202-206``).
    """

    @staticmethod
    def forward(ctx, flat, res, w_up, b_up, w_down, b_down, layer, logits):
        ctx.layer, ctx.has_res = layer, res is not None
        cfg, prep = layer.cfg, layer._get_prepared()
        out, routing, h_pre = ops.moe_forward_train(
            flat, cfg.top_k, prep["w_up"], prep["w_down"], prep["b_up"], prep["b_down"], cfg.activation,
            logits=logits, router_weight=layer.router_weight.detach() if logits is None else None,
            router_bias=layer.router_bias.detach() if logits is None else None, residual=res,
            workspace=layer._workspace)
        layer.last_routing = routing
        ctx.save_for_backward(flat, logits if logits is not None else flat.new_empty(0), h_pre)
        ctx.has_logits = logits is not None
        return out

    @staticmethod
    def backward(ctx, dout):
        flat, logits, h_pre = ctx.saved_tensors
        layer = ctx.layer
        cfg = layer.cfg
        prep, adj = layer._get_prepared(), layer._get_adjoint()
        use_logits = ctx.has_logits
        dx, dWu, dbu, dWd, dbd, _ = ops.moe_backward(
            flat, cfg.top_k, prep["w_up"], adj["w_up"], prep["w_down"], adj["w_down"], dout.contiguous(),
            prep["b_up"], prep["b_down"], cfg.activation, logits=logits if use_logits else None,
            router_weight=None if use_logits else layer.router_weight.detach(),
            router_bias=None if use_logits else layer.router_bias.detach(), routing_grad=False, h_pre=h_pre)
        return dx, (dout if ctx.has_res else None), dWu, dbu, dWd, dbd, None, None


class CliffordLinear(nn.Module):
    """CliffordLinear (clifford_linear.py:84-123) on the GPU: y = W * x + b per output channel."""

    def __init__(self, d_in: int, d_out: int, bias: bool = True, dtype: torch.dtype = torch.float32, device=None):
        super().__init__()
        self.d_in, self.d_out, self.dtype = d_in, d_out, dtype
        self.weight = nn.Parameter(xavier_clifford_init(d_out, d_in))
        self.bias = nn.Parameter(torch.zeros(d_out, 8)) if bias else None
        self._prep = None
        if device is not None:
            self.to(device)

    def _prepared(self):
        key = (self.weight._version, None if self.bias is None else self.bias._version, self.weight.device)
        if self._prep is None or self._prep[0] != key:
            fmt = "f32" if self.dtype == torch.float32 else "bf16"
            self._prep = (key, ops.prepare_weights(self.weight.detach().unsqueeze(0), fmt),
                          ops.prepare_bias(self.bias.detach().unsqueeze(0)) if self.bias is not None else None)
        return self._prep

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        batch = x.shape[:-2]
        flat = ops.to_mask_order(x.reshape(-1, self.d_in, 8).to(self.dtype))
        _, pw, pb = self._prepared()
        offsets = torch.tensor([0, flat.shape[0]], device=x.device, dtype=torch.int32)
        y = ops.grouped_clifford_linear(flat, pw, offsets, pb, "none", out_dtype=self.dtype)
        return y.reshape(*batch, self.d_out, 8)


class CliffordLayerNorm(nn.Module):
    """CliffordLayerNorm (``normalization.py:19-67``): y = gamma x_hat + beta (geometric product).

    gamma starts as the scalar 1 and beta at zero, as in the reference
    (``normalization.py:33-41``).  x: (..., d, 8), fp32 or bf16.
    """

    def __init__(self, d_model: int, eps: float = 1e-6, device=None):
        super().__init__()
        self.d_model, self.eps = d_model, eps
        gamma = torch.zeros(d_model, 8)
        gamma[:, 0] = 1.0
        self.gamma = nn.Parameter(gamma)
        self.beta = nn.Parameter(torch.zeros(d_model, 8))
        if device is not None:
            self.to(device)

    def forward(self, x: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        return ops.clifford_layer_norm(x.contiguous(), self.gamma.detach(), self.beta.detach(), self.eps,
                                       out_dtype=out_dtype)


class CliffordMoEBlockFFN(nn.Module):
    """The FFN half of ``HLMBlock.forward`` (``hlm_block.py:144-151``): ``x + moe(ffn_norm(x))``.

    With the energy router or caller logits the whole sub-layer is one library
    call (``ygg_moe_block_ffn``): the norm, then the MoE layer on the normed
    tokens with x added back in its combine.  Inference only: its output
    carries no autograd graph.
    """

    def __init__(self, cfg: MoEHLMConfig, device=None, generator: torch.Generator | None = None,
                 norm_eps: float = 1e-6):
        super().__init__()
        self.cfg = cfg
        self.ffn_norm = CliffordLayerNorm(cfg.d_model, norm_eps, device=device)
        self.moe = CliffordMoELayer(cfg, device=device, generator=generator)
        self._workspace = None

    @torch.no_grad()
    def load_reference_checkpoint(self, path: str, ffn_norm_index: int, grade_quant=None):
        """Load the FFN half of one ``HLMBlock`` from a reference checkpoint.

        Any of the reference's ``.npz`` layouts (``checkpoint.read_reference_checkpoint``);
        ``ffn_norm_index`` is the position of the block's ``ffn_norm.gamma`` in
        ``model.parameters()``, the rest follows ``HLMBlock.parameters()``
        (``hlm_block.py:230-241``).
        """
        from .checkpoint import hlm_block_ffn_state, read_reference_checkpoint

        st = hlm_block_ffn_state(read_reference_checkpoint(path), ffn_norm_index, self.cfg.n_experts)
        if st["w_up"].shape[1:3] != (self.cfg.d_ff, self.cfg.d_model):
            raise ValueError(f"checkpoint experts are {st['w_up'].shape[1:3]}, layer is "
                             f"{(self.cfg.d_ff, self.cfg.d_model)}")
        self.ffn_norm.gamma.copy_(torch.from_numpy(st["gamma"]))
        self.ffn_norm.beta.copy_(torch.from_numpy(st["beta"]))
        self.moe.load_reference_weights(router_weight=st["router_weight"], router_bias=st["router_bias"],
                                        w_up=st["w_up"], b_up=st["b_up"], w_down=st["w_down"], b_down=st["b_down"],
                                        grade_quant=grade_quant)

    def forward(self, x: torch.Tensor, logits: torch.Tensor | None = None) -> torch.Tensor:
        """x (B, T, d, 8) -> (B, T, d, 8)."""
        cfg, moe = self.cfg, self.moe
        if x.dim() != 4 or x.shape[-1] != 8 or x.shape[-2] != cfg.d_model:
            raise ValueError(f"expected (B, T, {cfg.d_model}, 8), got {tuple(x.shape)}")
        if x.dtype != cfg.dtype:
            raise ValueError(f"layer dtype is {cfg.dtype}, input is {x.dtype}")
        if cfg.router == "clifford_head" and logits is None:
            with torch.no_grad():  # the block is inference-only (the norm has no backward here)
                x_norm = self.ffn_norm(x)
                return moe.moe_forward(x_norm, logits=moe._head_logits(
                    x_norm.reshape(-1, cfg.d_model, 8), moe._get_prepared()), residual=x)
        if cfg.router == "logits" and logits is None:
            raise ValueError("router='logits' needs logits")
        B, T = x.shape[:2]
        flat = x.reshape(B * T, cfg.d_model, 8).contiguous()
        prep = moe._get_prepared()
        if logits is not None:
            logits = logits.reshape(B * T, cfg.n_experts).float().contiguous()
        ws_bytes = ops.moe_block_ffn_workspace_bytes(B * T, cfg.d_model, cfg.d_ff, cfg.n_experts, cfg.top_k,
                                                     cfg.dtype, cfg.weight_format)
        if self._workspace is None or self._workspace.numel() < ws_bytes or self._workspace.device != x.device:
            self._workspace = torch.empty((max(ws_bytes, 1),), device=x.device, dtype=torch.uint8)
        out, routing = ops.moe_block_ffn(
            flat, cfg.top_k, self.ffn_norm.gamma.detach(), self.ffn_norm.beta.detach(), prep["w_up"],
            prep["w_down"], prep["b_up"], prep["b_down"], cfg.activation, logits=logits,
            router_weight=moe.router_weight.detach() if logits is None else None,
            router_bias=moe.router_bias.detach() if logits is None else None, norm_eps=self.ffn_norm.eps,
            workspace=self._workspace)
        moe.last_routing = routing
        return out.reshape(B, T, cfg.d_model, 8)
