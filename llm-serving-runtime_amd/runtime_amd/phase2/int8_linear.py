"""Weight-only int8 linear (W8A16) for the quantized-linear slot.

The reference fills this slot with autoawq's int4 ``WQLinear``:
``PHASE2_QUANT=int4`` (``runtime/phase2/worker_server.py:126-128``) loads
``AutoAWQForCausalLM.from_quantized(...)`` (``:194-205``), whose modules keep
the ``nn.Linear`` contract ``y[..., N] = x[..., K] W^T (+ b)`` inside every HF
decoder layer. This module keeps that contract with a build-defined int8
format (per-output-channel symmetric absmax, fp16 scales; see the C ABI in
``include/mxdecode.h``) and runs the HIP kernels of libmxdecode:
``mx_w8a16_quantize`` + ``mx_w8a16_pack`` at load, ``mx_w8a16_linear`` per call.

``quantize_model_`` is the ``PHASE2_QUANT=int8`` counterpart of the reference's
AWQ load: it swaps the decoder-layer projections of an HF model in place.
"""

from __future__ import annotations

import threading

import torch
from torch import nn

from . import _hip

TILE_N = 16
TILE_K = 64

DEFAULT_TARGETS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

# Split-K partials of mx_w8a16_linear: one growable buffer per device, shared by
# every call on that device (calls on one stream are serialised; concurrent
# streams must not use this module's cache at the same time). A buffer that is
# outgrown stays allocated: graphs captured while it was current keep its address.
_workspaces: dict[torch.device, torch.Tensor] = {}
_retired: list[torch.Tensor] = []
_ws_lock = threading.Lock()


def _workspace(device: torch.device, nbytes: int) -> tuple[int | None, int]:
    if nbytes == 0:
        return None, 0
    with _ws_lock:
        ws = _workspaces.get(device)
        if ws is None or ws.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("int8 linear workspace must be sized before graph capture; "
                                   "run the step once eagerly")
            if ws is not None:
                _retired.append(ws)
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _workspaces[device] = ws
    return ws.data_ptr(), ws.numel()


def quantize_weight(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize ``weight [N, K]`` on the device: returns ``(q int8 [N, K], scale fp16 [N])``.

    Bit-exact with the CPU restatement of the format. Raises ValueError on
    non-finite weights (one host sync; this runs at model load).
    """
    _hip.require_device_tensor(weight, "weight")
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D [N, K], got {tuple(weight.shape)}")
    n, k = weight.shape
    w = weight.detach().to(torch.float32).contiguous()
    q = torch.empty((n, k), dtype=torch.int8, device=w.device)
    s = torch.empty((n,), dtype=torch.float16, device=w.device)
    lib = _hip.load()
    with torch.cuda.device(w.device):
        _hip.check(
            lib.mx_w8a16_quantize(w.data_ptr(), n, k, q.data_ptr(), s.data_ptr(), _hip.stream_handle(w.device)),
            "mx_w8a16_quantize",
        )
    if bool(torch.isnan(s).any()):
        raise ValueError("weight contains non-finite values")
    return q, s


def pack_weight(q: torch.Tensor) -> torch.Tensor:
    """Pack ``q int8 [N, K]`` into the kernels' 1 KiB tile layout (uint8 ``[N*K]``)."""
    _hip.require_device_tensor(q, "q")
    if q.dtype != torch.int8 or q.dim() != 2:
        raise ValueError("q must be a 2-D int8 tensor")
    n, k = q.shape
    if n % TILE_N or k % TILE_K:
        raise ValueError(f"int8 linear needs out_features % {TILE_N} == 0 and in_features % {TILE_K} == 0, got {n}x{k}")
    q = q.contiguous()
    packed = torch.empty((n * k,), dtype=torch.uint8, device=q.device)
    lib = _hip.load()
    with torch.cuda.device(q.device):
        _hip.check(lib.mx_w8a16_pack(q.data_ptr(), n, k, packed.data_ptr(), _hip.stream_handle(q.device)),
                   "mx_w8a16_pack")
    return packed


def int8_linear(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
                out_features: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """``y = x @ (q * s)^T + b`` for fp16 ``x [..., K]`` -> fp16 ``[..., N]``."""
    _hip.require_device_tensor(x, "x")
    if x.dtype != torch.float16:
        raise ValueError(f"int8 linear expects fp16 activations, got {x.dtype}")
    k = int(x.shape[-1])
    n = int(out_features)
    if packed.numel() != n * k:
        raise ValueError(f"packed weight has {packed.numel()} bytes, expected {n}x{k}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    m = int(x2.shape[0])
    if out is None:
        y = torch.empty((m, n), dtype=torch.float16, device=x.device)
    else:
        y = out.view(m, n)
    if m == 0:
        return y.view(*lead, n)
    lib = _hip.load()
    ws_ptr, ws_bytes = _workspace(x.device, int(lib.mx_w8a16_workspace_bytes(m, n, k)))
    _hip.check(
        lib.mx_w8a16_linear(
            x2.data_ptr(), m, k, x2.stride(0), packed.data_ptr(), scale.data_ptr(),
            bias.data_ptr() if bias is not None else None, y.data_ptr(), n, y.stride(0),
            ws_ptr, ws_bytes, _hip.stream_handle(x.device),
        ),
        "mx_w8a16_linear",
    )
    return y.view(*lead, n)


def linear_splits(m: int, n: int, k: int) -> int:
    """K splits the MFMA kernel uses for ``[m, k] x [k, n]`` (1: :func:`int8_linear` writes y directly)."""
    return int(_hip.load().mx_w8a16_splits(m, n, k))


def gateup_fusable(m: int, n: int, k: int) -> bool:
    """Whether :func:`int8_gateup_swiglu` takes ``m`` rows of a ``[n, k]`` gate||up weight: any
    ``m >= 1`` (its launches never split K; ``n`` a multiple of 16, ``k`` of 64)."""
    return m >= 1 and n % 16 == 0 and k % 64 == 0


def int8_linear_partials(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, out_features: int,
                         partials: torch.Tensor) -> int:
    """Split-K partials of ``x @ (q*s)^T`` into fp32 ``partials`` (``[splits, M, N]`` contiguous, or larger).

    Returns the split count. Summing the splits, adding the bias and rounding
    to fp16 gives :func:`int8_linear`'s output; the decode glue kernels do that
    in their input stage (``mx_*_splits``), so no reduce launch is needed.
    """
    _hip.require_device_tensor(x, "x")
    if x.dtype != torch.float16 or x.dim() != 2:
        raise ValueError("int8_linear_partials expects fp16 x [M, K]")
    m, k = (int(v) for v in x.shape)
    n = int(out_features)
    if x.stride(-1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    if partials.dtype != torch.float32 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous fp32 tensor")
    lib = _hip.load()
    splits = int(lib.mx_w8a16_splits(m, n, k))
    _hip.check(lib.mx_w8a16_linear_partials(x.data_ptr(), m, k, x.stride(0), packed.data_ptr(), scale.data_ptr(), n,
                                            partials.data_ptr(), partials.numel() * 4, _hip.stream_handle(x.device)),
               "mx_w8a16_linear_partials")
    return splits


def _gate_up_rows(gate_up: torch.Tensor) -> torch.Tensor:
    _hip.require_device_tensor(gate_up, "gate_up")
    if gate_up.dtype != torch.float16 or gate_up.dim() != 2 or gate_up.shape[1] % 2:
        raise ValueError("gate_up must be fp16 [M, 2K]")
    if gate_up.stride(-1) != 1 or gate_up.stride(0) % 8 or gate_up.data_ptr() % 16:
        gate_up = gate_up.contiguous()
    return gate_up


def int8_linear_swiglu(gate_up: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
                       out_features: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """``y = (silu(g) * u) @ (q*s)^T + b`` for ``gate_up = [g | u]`` fp16 ``[M, 2K]``, 4 < M <= 128.

    The product is formed inside the GEMM's x staging (same rounding as
    ``mx_silu_mul``), so it is never written out.
    """
    gu = _gate_up_rows(gate_up)
    m, k = int(gu.shape[0]), int(gu.shape[1]) // 2
    n = int(out_features)
    y = torch.empty((m, n), dtype=torch.float16, device=gu.device) if out is None else out.view(m, n)
    lib = _hip.load()
    ws_ptr, ws_bytes = _workspace(gu.device, int(lib.mx_w8a16_workspace_bytes(m, n, k)))
    _hip.check(lib.mx_w8a16_linear_swiglu(gu.data_ptr(), m, k, gu.stride(0), packed.data_ptr(), scale.data_ptr(),
                                          bias.data_ptr() if bias is not None else None, y.data_ptr(), n, y.stride(0),
                                          ws_ptr, ws_bytes, _hip.stream_handle(gu.device)), "mx_w8a16_linear_swiglu")
    return y


def int8_linear_partials_swiglu(gate_up: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, out_features: int,
                                partials: torch.Tensor) -> int:
    """:func:`int8_linear_partials` with the SwiGLU product of ``gate_up`` as x; returns the split count."""
    gu = _gate_up_rows(gate_up)
    m, k = int(gu.shape[0]), int(gu.shape[1]) // 2
    n = int(out_features)
    if partials.dtype != torch.float32 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous fp32 tensor")
    lib = _hip.load()
    splits = int(lib.mx_w8a16_splits(m, n, k))
    _hip.check(lib.mx_w8a16_linear_partials_swiglu(gu.data_ptr(), m, k, gu.stride(0), packed.data_ptr(),
                                                   scale.data_ptr(), n, partials.data_ptr(), partials.numel() * 4,
                                                   _hip.stream_handle(gu.device)), "mx_w8a16_linear_partials_swiglu")
    return splits


def gateup_interleave(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Stack gate and up rows (``[I, ...]`` each) in alternating groups of 8, the row order
    ``mx_w8a16_gateup_swiglu`` expects: rows 16t + [0, 8) = gate 8t + [0, 8), rows
    16t + [8, 16) = up 8t + [0, 8). Works for weights ``[I, K]`` and for scales/biases ``[I]``."""
    if gate.shape != up.shape or gate.shape[0] % 8:
        raise ValueError("gate and up must have the same shape with a multiple of 8 rows")
    i = gate.shape[0]
    rest = tuple(gate.shape[1:])
    return torch.stack((gate.reshape(i // 8, 8, *rest), up.reshape(i // 8, 8, *rest)), dim=1).reshape(2 * i, *rest)


def gateup_deinterleave(y: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`gateup_interleave` on the last dimension: ``[..., 2I]`` -> ``[gate | up]``."""
    lead, n = y.shape[:-1], y.shape[-1]
    return y.reshape(*lead, n // 16, 2, 8).transpose(-3, -2).reshape(*lead, n)


def int8_gateup_swiglu(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
                       inter: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(x W_gate^T) * (x W_up^T)`` from an interleaved gate||up weight, as fp16 ``[M, inter]``."""
    _hip.require_device_tensor(x, "x")
    if x.dtype != torch.float16 or x.dim() != 2:
        raise ValueError("int8_gateup_swiglu expects fp16 x [M, K]")
    if x.stride(-1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    m, k = int(x.shape[0]), int(x.shape[1])
    y = torch.empty((m, inter), dtype=torch.float16, device=x.device) if out is None else out.view(m, inter)
    _hip.check(_hip.load().mx_w8a16_gateup_swiglu(
        x.data_ptr(), m, k, x.stride(0), packed.data_ptr(), scale.data_ptr(),
        bias.data_ptr() if bias is not None else None, y.data_ptr(), inter, y.stride(0),
        _hip.stream_handle(x.device)), "mx_w8a16_gateup_swiglu")
    return y


MLP_SYNC_WORDS = 64  # int32 words of a fused MLP launch's sync buffer
MLP_SYNC_ERR = 33    # the word holding its error bits


def mlp_fusable(m: int, hidden: int, inter: int, out_features: int) -> bool:
    """Whether :func:`int8_mlp_fused_partials` takes ``m`` rows of this MLP on the current device."""
    return bool(_hip.load().mx_w8a16_mlp_fused_supported(m, hidden, inter, out_features))


def int8_mlp_fused_partials(x: torch.Tensor, gate_up: tuple, down: tuple, act: torch.Tensor, partials: torch.Tensor,
                            sync: torch.Tensor) -> int:
    """:func:`int8_gateup_swiglu` into ``act`` and :func:`int8_linear_partials` of ``act`` with the down
    weight into ``partials``, as one launch (``mx_w8a16_mlp_fused_partials``); bit-identical to the two
    calls. ``gate_up`` = (packed, scale, 2 * inter, bias) with interleaved rows, ``down`` = (packed, scale,
    out_features, ...); ``act`` fp16 [M, inter] with 128-byte aligned rows; ``sync`` int32 [64] zeros,
    kept between calls. Returns down's split count."""
    _hip.require_device_tensor(x, "x")
    if x.dtype != torch.float16 or x.dim() != 2:
        raise ValueError("int8_mlp_fused_partials expects fp16 x [M, K]")
    if x.stride(-1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    m, k = (int(v) for v in x.shape)
    gpk, gsc, gn, gbias = gate_up[0], gate_up[1], int(gate_up[2]), gate_up[3]
    dpk, dsc, n = down[0], down[1], int(down[2])
    inter = gn // 2
    if act.dtype != torch.float16 or act.dim() != 2 or tuple(act.shape) != (m, inter) or act.stride(-1) != 1:
        raise ValueError(f"act must be fp16 [{m}, {inter}] with unit column stride")
    if partials.dtype != torch.float32 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous fp32 tensor")
    if sync.dtype != torch.int32 or sync.numel() < MLP_SYNC_WORDS or not sync.is_contiguous():
        raise ValueError(f"sync must be a contiguous int32 tensor of at least {MLP_SYNC_WORDS} words")
    lib = _hip.load()
    _hip.check(lib.mx_w8a16_mlp_fused_partials(
        x.data_ptr(), m, k, x.stride(0), gpk.data_ptr(), gsc.data_ptr(), gbias.data_ptr() if gbias is not None else None,
        inter, act.data_ptr(), act.stride(0), dpk.data_ptr(), dsc.data_ptr(), n, partials.data_ptr(),
        partials.numel() * 4, sync.data_ptr(), _hip.stream_handle(x.device)), "mx_w8a16_mlp_fused_partials")
    return int(lib.mx_w8a16_splits(m, n, inter))


class Int8Linear(nn.Module):
    """Drop-in for ``nn.Linear`` on the decode path with int8 weights and fp16 scales."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 device: torch.device | str | None = None) -> None:
        super().__init__()
        if out_features % TILE_N or in_features % TILE_K:
            raise ValueError(
                f"Int8Linear needs out_features % {TILE_N} == 0 and in_features % {TILE_K} == 0, "
                f"got {out_features}x{in_features}"
            )
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.register_buffer("packed_weight", torch.zeros(out_features * in_features, dtype=torch.uint8, device=device))
        self.register_buffer("weight_scale", torch.ones(out_features, dtype=torch.float16, device=device))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16, device=device))
        else:
            self.bias = None

    @classmethod
    def from_linear(cls, linear: nn.Linear, device: torch.device | str | None = None) -> "Int8Linear":
        dev = torch.device(device) if device is not None else linear.weight.device
        if dev.type != "cuda":
            raise ValueError("Int8Linear.from_linear quantizes on a ROCm device; pass device='cuda'")
        mod = cls(linear.in_features, linear.out_features, bias=linear.bias is not None, device=dev)
        q, s = quantize_weight(linear.weight.detach().to(dev))
        mod.packed_weight.copy_(pack_weight(q))
        mod.weight_scale.copy_(s)
        if linear.bias is not None:
            mod.bias.copy_(linear.bias.detach().to(dev, torch.float16))
        return mod

    @classmethod
    def from_quantized(cls, q: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None = None) -> "Int8Linear":
        n, k = q.shape
        mod = cls(k, n, bias=bias is not None, device=q.device)
        mod.packed_weight.copy_(pack_weight(q))
        mod.weight_scale.copy_(scale.to(torch.float16))
        if bias is not None:
            mod.bias.copy_(bias.to(torch.float16))
        return mod

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return int8_linear(x, self.packed_weight, self.weight_scale, self.bias, self.out_features)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}, int8"


def quantize_model_(model: nn.Module, targets: tuple[str, ...] = DEFAULT_TARGETS, include_lm_head: bool = False,
                    device: torch.device | str | None = None) -> nn.Module:
    """Replace the named ``nn.Linear`` projections of ``model`` with :class:`Int8Linear` in place."""
    replace: list[tuple[nn.Module, str, nn.Linear]] = []
    for parent in model.modules():
        for name, child in parent.named_children():
            if isinstance(child, nn.Linear) and (name in targets or (include_lm_head and name == "lm_head")):
                replace.append((parent, name, child))
    for parent, name, child in replace:
        setattr(parent, name, Int8Linear.from_linear(child, device=device))
    return model
