"""A complete single-GPU MoE feed-forward block with matched implementation variants.

Mirrors ``src/moe_dispatch/layer.py:12-214``: ``MoEConfig``, ``MoEWeights``,
``make_weights``, ``LayerWorkspace``, ``MoEBlock`` (``route``, ``workspace``,
``experts_forward``, ``forward``, ``set_routing_pattern``) and
``token_major_oracle``. Implementations:

* ``cuda_fused``: HIP fused router (fp32 logits + bias + top-k + softmax),
  HIP dispatch, HIP gate/up GEMM with the SwiGLU epilogue, HIP down GEMM, HIP
  combine. The drop-in for the reference's ``cuda_fused``.
* ``cuda``: PyTorch router, HIP transport, HIP GEMMs with a separate
  PyTorch SwiGLU.
* ``torch``: the PyTorch variant (CPU or GPU), used as the baseline.

Top-k may be 1..8 (the reference allows 1 or 2); ``set_routing_bias`` sets an
arbitrary router bias.
"""

from dataclasses import dataclass
import math

import torch

from . import _lib
from ._extension import current_stream_handle, get_extension, weight_row_stride
from .experts import grouped_linear, resolve_backend, swiglu_reference
from .reference import TorchWorkspace
from .workspace import MAX_EXPERTS, MAX_TOPK, CudaWorkspace

IMPLEMENTATIONS = ("torch", "cuda", "cuda_fused")


@dataclass(frozen=True)
class MoEConfig:
    hidden: int = 512
    intermediate: int = 1024
    experts: int = 8
    topk: int = 2
    alignment: int = 8

    def __post_init__(self):
        if self.hidden < 8 or self.intermediate < 8:
            raise ValueError("hidden/intermediate must be at least 8")
        if self.hidden % 8 or self.intermediate % 8:
            raise ValueError("grouped GEMM dimensions must be multiples of 8")
        if (
            not 1 <= self.experts <= MAX_EXPERTS
            or not 1 <= self.topk <= MAX_TOPK
            or self.topk > self.experts
        ):
            raise ValueError("invalid expert/topk configuration")
        if not 8 <= self.alignment <= 128 or self.alignment % 8:
            raise ValueError("full-block grouped GEMM alignment must be a multiple of 8 up to 128")


@dataclass
class MoEWeights:
    router: torch.Tensor
    gate_up: torch.Tensor
    down: torch.Tensor


def _capturing():
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def make_weights(config, device, dtype, seed=42):
    """Seeded weights, drawn in the reference's order (``layer.py:38-59``).

    router ``[E,H]`` fp32 ~ N(0,1/H); gate_up ``[E,2I,H]`` ~ N(0,1/H) and down
    ``[E,H,I]`` ~ N(0,1/I), both cast to ``dtype``.
    """
    generator = torch.Generator(device=device).manual_seed(seed)
    e, h, i = config.experts, config.hidden, config.intermediate
    router = torch.randn(e, h, device=device, generator=generator) / math.sqrt(h)
    gate_up = (torch.randn(e, 2 * i, h, device=device, generator=generator) / math.sqrt(h)).to(dtype)
    down = (torch.randn(e, h, i, device=device, generator=generator) / math.sqrt(i)).to(dtype)
    return MoEWeights(router, gate_up, down)


# Elements of padding after each gate/up weight row whose length is a power
# of two bytes of at least 8 KiB (H = 4096, 8192, ...), for the fused block.
# The weight-streaming GEMMs read every row of a tile at the same k offset at
# once, and rows a power of two apart then fall on the same memory channels.
# Measured at H = 4096, I = 14336, 8 experts, top-2, alternating on one box:
# padded rows make the gate/up GEMM 11% faster at 1 token and 10% at 16
# (91.8 -> 82.1 and 337.8 -> 304.7 us; forwards 165 -> 154.5 and 527 -> 495
# us) and leave it unchanged at 4096 tokens. At H = 2048 (4 KiB rows; 8192
# tokens, 64 experts, top-6) the gathered gate/up GEMM ran 1% slower with
# padded rows, so those are not padded. The results are the same bit for bit
# (each output is the same MFMA chain). The down GEMM's rows (I = 14336) are
# not a power of two apart.
GATE_UP_ROW_PADDING = 64


def padded_gate_up(weight):
    """``weight`` ([E, 2I, H]) as a ``[:, :, :H]`` view of row-padded storage when
    its rows are a power of two bytes of at least 8 KiB long, else contiguous."""
    row_bytes = weight.shape[2] * weight.element_size()
    if row_bytes < 8192 or row_bytes & (row_bytes - 1):
        return weight.contiguous()
    e, n, k = weight.shape
    storage = torch.zeros(e, n, k + GATE_UP_ROW_PADDING, device=weight.device, dtype=weight.dtype)
    storage[:, :, :k].copy_(weight)
    return storage[:, :, :k]


@dataclass
class LayerWorkspace:
    transport: object
    projection: torch.Tensor
    activated: torch.Tensor
    expert_output: torch.Tensor


class MoEBlock(torch.nn.Module):
    """Inference-only top-k MoE: router, dispatch, two grouped GEMMs, SwiGLU, combine.

    Output is a reusable view: clone it before the next call.
    """

    def __init__(
        self,
        config=None,
        *,
        device="cuda",
        dtype=torch.bfloat16,
        implementation="cuda_fused",
        expert_backend="auto",
        seed=42,
        weights=None,
    ):
        super().__init__()
        self.config = config or MoEConfig()
        if implementation not in IMPLEMENTATIONS:
            raise ValueError("implementation must be torch, cuda, or cuda_fused")
        device = torch.device(device)
        if implementation != "torch" and device.type != "cuda":
            raise RuntimeError("HIP implementations require a GPU")
        if device.type == "cuda" and dtype != torch.bfloat16:
            raise ValueError("full GPU block uses BF16 grouped GEMMs")
        self.implementation = implementation
        backend = resolve_backend(device, expert_backend)
        if implementation != "torch" and backend != "hip":
            raise ValueError("HIP implementations use the HIP grouped GEMM (expert_backend='hip')")
        self.expert_backend = backend
        weights = weights or make_weights(self.config, device, dtype, seed)
        cfg = self.config
        if weights.gate_up.shape != (cfg.experts, 2 * cfg.intermediate, cfg.hidden) or (
            weights.down.shape != (cfg.experts, cfg.hidden, cfg.intermediate)
        ):
            raise ValueError("expert weights do not match the block configuration")
        if weights.router.shape != (cfg.experts, cfg.hidden):
            raise ValueError("router weights do not match the block configuration")
        self.register_buffer("router_weight", weights.router.contiguous())
        # The fused block keeps power-of-two gate/up rows padded (GATE_UP_ROW_PADDING);
        # the tensor is a view of that storage, so in-place updates reach the kernels.
        gate_up = padded_gate_up(weights.gate_up) if implementation == "cuda_fused" else weights.gate_up.contiguous()
        self.register_buffer("gate_up_weight", gate_up)
        self.register_buffer("down_weight", weights.down.contiguous())
        self.register_buffer("routing_bias", torch.zeros(cfg.experts, device=device))
        self._workspaces = {}
        self._route_buffers = {}
        self._router_scratch = None  # bf16 split of the router weights (fused router)
        self._router_split_of = None  # _router_split_key() of the weights the split holds
        self._split_in_capture = True  # record the router split into captured graphs
        self._launches = {}  # cuda_fused: pre-validated launches per input signature
        self._extension = get_extension() if implementation != "torch" else None

    def set_routing_pattern(self, pattern):
        if pattern not in ("balanced", "skewed"):
            raise ValueError("routing pattern must be balanced or skewed")
        self.routing_bias.zero_()
        if pattern == "skewed":
            self.routing_bias[: self.config.topk] = 5.0

    def set_routing_bias(self, bias):
        """Set an arbitrary fp32 router bias ``[E]`` (e.g. a Zipf-shaped skew)."""
        bias = torch.as_tensor(bias, dtype=torch.float32)
        if bias.shape != (self.config.experts,):
            raise ValueError("routing bias must have shape [experts]")
        self.routing_bias.copy_(bias)

    def route(self, x):
        return self._route(x)

    def _route(self, x, ranked_into=None):
        """route(); with a CudaWorkspace whose shape has a ranked route
        (``rank_tile`` > 0), the fused router also writes that workspace's
        in-tile ranks and tile counts for its ``dispatch_ranked``."""
        if self.implementation == "cuda_fused":
            key = (x.shape[0], x.device)
            if key not in self._route_buffers:
                shape = (x.shape[0], self.config.topk)
                self._route_buffers[key] = (
                    torch.empty(shape, device=x.device, dtype=torch.int32),
                    torch.empty(shape, device=x.device, dtype=torch.int64),
                    torch.empty(shape, device=x.device, dtype=torch.float32),
                )
            ids32, ids64, weights = self._route_buffers[key]
            if self._router_scratch is None or self._router_scratch.device != x.device:
                need = self._extension.router_scratch_bytes(self.config.experts, self.config.hidden)
                self._router_scratch = torch.empty(need, dtype=torch.uint8, device=x.device)
                self._router_split_of = None
            router_weight, split_of = self._router_split_plan()
            weight = None if router_weight is None else self.router_weight
            if ranked_into is None:
                self._extension.router_fused_out(x, weight, self.routing_bias, ids32, ids64, weights,
                                                 scratch=self._router_scratch)
            else:
                self._extension.router_fused_ranked_out(x, weight, self.routing_bias, ids32, ids64, weights,
                                                        ranked_into.tile_ranks, ranked_into.tile_counts,
                                                        scratch=self._router_scratch)
            self._router_split_of = split_of
            return ids32, ids64, weights
        logits = torch.nn.functional.linear(x.float(), self.router_weight) + self.routing_bias
        selected, ids64 = torch.topk(logits, self.config.topk, dim=-1)
        weights = torch.softmax(selected, dim=-1).contiguous()
        return ids64.to(torch.int32).contiguous(), ids64.contiguous(), weights

    def _router_split_key(self):
        """Identity of the router weights the bf16 split was taken from.

        The key holds the tensor itself (so its storage cannot be freed and
        reused by another tensor at the same address while the key is kept),
        its address, version counter, dtype, shape and device. None when the
        tensor has no version counter (inference tensors): then every call splits.
        """
        w = self.router_weight
        try:
            version = w._version
        except RuntimeError:  # inference tensors do not count versions
            return None
        return (w, w.data_ptr(), version, w.dtype, tuple(w.shape), w.device)

    @staticmethod
    def _same_split(a, b):
        return a is not None and b is not None and a[0] is b[0] and a[1:] == b[1:]

    def _router_split_plan(self):
        """(router weight pointer or None, split key to record) for the next fused-router call.

        The bf16 split of the router weights is redone only when they may have
        changed (another tensor, or an in-place write, which bumps the version
        counter). Inside a graph capture it is recorded into the graph, so that
        every replay reads the weights as they are then, unless the capture is
        ``capture_forward``'s: its graph's replay() re-splits beforehand, and only
        when the weights changed. A recorded split runs only when the graph is
        replayed, so after recording one the split counts as stale.
        """
        split_of = self._router_split_key()
        capturing = _capturing()
        current = self._same_split(split_of, self._router_split_of)
        if current and not (capturing and self._split_in_capture):
            return None, split_of
        return self.router_weight.data_ptr(), (None if capturing else split_of)

    def workspace(self, x):
        key = (x.shape[0], x.dtype, x.device)
        if key not in self._workspaces:
            cfg = self.config
            common = (x.shape[0], cfg.hidden, cfg.experts, cfg.topk, x.dtype)
            if self.implementation == "torch":
                transport = TorchWorkspace(*common, device=x.device, alignment=cfg.alignment)
            else:
                transport = CudaWorkspace(
                    *common, device=x.device, alignment=cfg.alignment, extension=self._extension
                )
            rows = transport.capacity_rows
            # The fused gate/up kernel never materialises the [R, 2I] projection.
            proj_rows = 0 if self.implementation == "cuda_fused" else rows
            self._workspaces[key] = LayerWorkspace(
                transport,
                torch.empty((proj_rows, 2 * cfg.intermediate), device=x.device, dtype=x.dtype),
                torch.empty((rows, cfg.intermediate), device=x.device, dtype=x.dtype),
                torch.empty((rows, cfg.hidden), device=x.device, dtype=x.dtype),
            )
        return self._workspaces[key]

    def _experts_gathered(self, state, x):
        """experts_forward() with the gate/up GEMM reading x through
        ``transport.row_src`` (after dispatch_rows), not the packed rows."""
        transport = state.transport
        ext = self._extension
        ext.gateup_swiglu_gathered_out(x, transport.row_src, self.gate_up_weight, transport.offsets, state.activated)
        ext.grouped_gemm_out(state.activated, self.down_weight, transport.offsets, state.expert_output)
        return state.expert_output

    def experts_forward(self, state):
        transport = state.transport
        offsets = transport.offsets
        if self.implementation == "cuda_fused":
            ext = self._extension
            ext.gateup_swiglu_out(transport.packed, self.gate_up_weight, offsets, state.activated)
            ext.grouped_gemm_out(state.activated, self.down_weight, offsets, state.expert_output)
            return state.expert_output
        ends = offsets[1:]
        grouped_linear(
            transport.packed, self.gate_up_weight, ends, backend=self.expert_backend,
            output=state.projection, offsets=offsets,
        )
        state.activated.copy_(swiglu_reference(state.projection))
        grouped_linear(
            state.activated, self.down_weight, ends, backend=self.expert_backend,
            output=state.expert_output, offsets=offsets,
        )
        return state.expert_output

    @torch.inference_mode()
    def forward(self, x):
        if x.ndim != 2 or x.shape[1] != self.config.hidden or not x.is_contiguous():
            raise ValueError("expected contiguous x[T,hidden]")
        if x.dtype != self.gate_up_weight.dtype or x.device != self.gate_up_weight.device:
            raise ValueError("input dtype/device must match expert weights")
        if x.shape[0] == 0:
            return torch.empty_like(x)
        if self.implementation == "cuda_fused":
            launches = self._launches.get((x.shape[0], x.device))
            if launches is not None and launches.still_valid(self):
                return launches(self, x)
        state = self.workspace(x)
        fused = self.implementation == "cuda_fused"
        # The fused router does the dispatch's counting pass when the shape allows.
        ranked = fused and state.transport.rank_tile > 0
        gathered = fused and _gathers(x, self.config.topk)
        ids32, ids64, weights = self._route(x, state.transport if ranked else None)
        transport = state.transport
        if gathered:
            # No packed copy: the gate/up GEMM reads x through the row table.
            if ranked:
                transport.dispatch_ranked_rows(ids32)
            else:
                transport.dispatch_rows(ids32)
            output = self._experts_gathered(state, x)
        else:
            if ranked:
                transport.dispatch_ranked(x, ids32)
            else:
                transport.dispatch(x, ids32, ids64)
            output = self.experts_forward(state)
        transport.combine(output, weights)
        if self.implementation == "cuda_fused":
            # Every operator above validated its tensors; later calls of this
            # shape reuse the checked arguments.
            self._launches[(x.shape[0], x.device)] = _FusedLaunches(self, x, state)
        return state.transport.output


def _gathers(x, topk):
    """Whether the fused forward skips the packed copy, the gate/up GEMM reading
    x through the dispatch's row table. It needs the ring kernels (hidden a
    multiple of 64) and x below 2 GiB, and pays off from top-3 on: the gathered
    GEMM is 1-2% slower than the packed one (H=4096, I=14336, E=8: 1510 against
    1489 us; H=1024, I=2048, E=16: +2.2%), which at top-2 costs about what the
    copy does, while with K rows per token the copy it saves grows with K
    (H=2048, I=1408, E=64, top-6: dispatch 39 -> 7 us, forward -3.8%). With
    that configuration's Zipf routing the gathered GEMM is itself faster than
    the packed one (560 against 638 us): it reads x's 33.6 MB where the packed
    kernel reads a 201 MB copy."""
    return topk >= 3 and x.shape[1] % 64 == 0 and x.numel() * x.element_size() < 2**31


class _FusedLaunches:
    """The C-ABI calls of one validated cuda_fused forward, for reuse.

    A forward through the validating operators (router_fused_out, dispatch,
    the two grouped GEMMs, combine) fixes every argument but x's address and
    the stream: workspace and weight pointers, sizes, the dtype code. Later
    forwards of the same token count on the same device make the same five
    calls with those arguments while every parameter tensor the calls read is
    the object it was, at the same address, with the same dtype, shape and
    layout (an in-place update keeps all of these; the router split follows
    the weights' version as in ``MoEBlock.route``). Anything else sends the
    forward back through the validating path, which raises on a bad tensor.
    This removes about 50 us of host work per forward (validation and stream
    lookups), which dominates the eager latency of small batches.
    """

    _PARAMETERS = ("router_weight", "gate_up_weight", "down_weight", "routing_bias", "_router_scratch")

    def __init__(self, block, x, state):
        cfg = block.config
        t = state.transport
        ids32, ids64, weights = block._route_buffers[(x.shape[0], x.device)]
        self.lib = block._extension.lib
        self.device_index = x.device.index if x.device.index is not None else torch.cuda.current_device()
        self.fingerprint = self._fingerprint(block)
        self.keep = (ids32, ids64, weights, t, state)  # the buffers below stay allocated
        tokens, hidden = x.shape
        rows = t.packed.shape[0]
        scratch = block._router_scratch
        self.router = (block.routing_bias.data_ptr(), ids32.data_ptr(), ids64.data_ptr(), weights.data_ptr(),
                       None, scratch.data_ptr(), scratch.numel() * scratch.element_size(),
                       tokens, hidden, cfg.experts, cfg.topk)
        # A ranked route (the router counts for the dispatch) whenever the shape
        # has one, and the row table instead of the packed copy whenever the
        # gate/up GEMM can gather, as in forward().
        self.ranked = t.rank_tile > 0
        self.gathered = _gathers(x, cfg.topk)
        # The weights' row strides (contiguous, or gate/up rows padded); anything
        # else was refused by the validating forward that built these launches.
        gate_up_stride = weight_row_stride(block.gate_up_weight)
        down_stride = weight_row_stride(block.down_weight)
        if gate_up_stride is None or down_stride is None:
            raise RuntimeError("expert weights must be contiguous or row-padded")
        index = (ids32.data_ptr(), t.counts.data_ptr(), t.offsets.data_ptr(), t.slots.data_ptr())
        if self.ranked:
            self.router += (t.tile_ranks.data_ptr(), t.tile_counts.data_ptr(), t.tile_counts.numel() * 4)
            ranked_table = (t.tile_ranks.data_ptr(), t.tile_counts.data_ptr(), t.tile_counts.numel() * 4, t.rank_tile)
        if self.gathered:
            after = (t.inverse.data_ptr(), t.row_src.data_ptr())
            if self.ranked:
                self.dispatch = index + after + ranked_table + (tokens, cfg.experts, cfg.topk, t.alignment, rows)
            else:
                self.dispatch = index + after + (t.scratch.data_ptr(), t.scratch.numel() * t.scratch.element_size(),
                                                 tokens, cfg.experts, cfg.topk, t.alignment, rows)
            # moe_grouped_gateup_swiglu_gathered_strided after x.
            self.gateup = (t.row_src.data_ptr(), tokens, block.gate_up_weight.data_ptr(), gate_up_stride,
                           state.activated.data_ptr(), t.offsets.data_ptr(), rows, hidden, cfg.intermediate,
                           cfg.experts)
        else:
            packed = (t.packed.data_ptr(), t.inverse.data_ptr())
            if self.ranked:
                self.dispatch = (_lib.DTYPE_BF16,) + index + packed + ranked_table + (
                    tokens, hidden, cfg.experts, cfg.topk, t.alignment, rows, int(bool(t.vectorized)))
            else:
                self.dispatch = (_lib.DTYPE_BF16,) + index + packed + (
                    t.scratch.data_ptr(), t.scratch.numel() * t.scratch.element_size(), tokens, hidden, cfg.experts,
                    cfg.topk, t.alignment, rows, int(bool(t.vectorized)))
            self.gateup = (t.packed.data_ptr(), block.gate_up_weight.data_ptr(), gate_up_stride,
                           state.activated.data_ptr(), t.offsets.data_ptr(), rows, hidden, cfg.intermediate,
                           cfg.experts)
        self.down = (state.activated.data_ptr(), block.down_weight.data_ptr(), down_stride,
                     state.expert_output.data_ptr(), t.offsets.data_ptr(), rows, hidden, cfg.intermediate,
                     cfg.experts)
        self.combine = (state.expert_output.data_ptr(), _lib.DTYPE_BF16, t.inverse.data_ptr(), weights.data_ptr(),
                        t.output.data_ptr(), tokens, hidden, cfg.topk, rows)
        self.output = t.output
        if x.dtype != torch.bfloat16:
            raise RuntimeError("cuda_fused launches are bf16")

    @classmethod
    def _fingerprint(cls, block):
        tensors = tuple(getattr(block, name) for name in cls._PARAMETERS)
        return tensors, tuple((v.data_ptr(), v.dtype, tuple(v.shape), v.stride()) for v in tensors)

    def still_valid(self, block):
        tensors, described = self.fingerprint
        current = tuple(getattr(block, name) for name in self._PARAMETERS)
        if not all(a is b for a, b in zip(current, tensors)):
            return False
        return all((v.data_ptr(), v.dtype, tuple(v.shape), v.stride()) == d for v, d in zip(current, described))

    def __call__(self, block, x):
        lib = self.lib
        stream = current_stream_handle(self.device_index)
        x_ptr = x.data_ptr()
        router_weight, split_of = block._router_split_plan()
        if self.ranked:
            lib.check(lib.moe_router_fused_ranked(x_ptr, router_weight, *self.router, stream), "router_fused_out")
        else:
            lib.check(lib.moe_router_fused(x_ptr, router_weight, *self.router, stream), "router_fused_out")
        block._router_split_of = split_of
        if self.gathered:
            if self.ranked:
                lib.check(lib.moe_dispatch_ranked_rows(*self.dispatch, stream), "dispatch")
            else:
                lib.check(lib.moe_dispatch_rows(*self.dispatch, stream), "dispatch")
            lib.check(lib.moe_grouped_gateup_swiglu_gathered_strided(x_ptr, *self.gateup, stream),
                      "gateup_swiglu_out")
        else:
            if self.ranked:
                lib.check(lib.moe_dispatch_ranked(x_ptr, *self.dispatch, stream), "dispatch")
            else:
                lib.check(lib.moe_dispatch(x_ptr, *self.dispatch, stream), "dispatch")
            lib.check(lib.moe_grouped_gateup_swiglu_strided(*self.gateup, stream), "gateup_swiglu_out")
        lib.check(lib.moe_grouped_gemm_strided(*self.down, stream), "grouped_gemm_out")
        lib.check(lib.moe_combine(*self.combine, stream), "combine_out")
        return self.output

    def stage_calls(self, x):
        """Each stage of __call__ as a zero-argument callable on the current
        stream (the router with the split it holds), for per-stage timing."""
        lib, x_ptr = self.lib, x.data_ptr()

        def bind(name, *args):
            def run():
                lib.check(getattr(lib, name)(*args, current_stream_handle(self.device_index)), name)
            return run

        router = "moe_router_fused_ranked" if self.ranked else "moe_router_fused"
        if self.gathered:
            dispatch = bind("moe_dispatch_ranked_rows" if self.ranked else "moe_dispatch_rows", *self.dispatch)
            gateup = bind("moe_grouped_gateup_swiglu_gathered_strided", x_ptr, *self.gateup)
        else:
            dispatch = bind("moe_dispatch_ranked" if self.ranked else "moe_dispatch", x_ptr, *self.dispatch)
            gateup = bind("moe_grouped_gateup_swiglu_strided", *self.gateup)
        return {"router": bind(router, x_ptr, None, *self.router), "dispatch": dispatch, "gateup_swiglu": gateup,
                "down": bind("moe_grouped_gemm_strided", *self.down), "combine": bind("moe_combine", *self.combine)}


@torch.inference_mode()
def token_major_oracle(block, x):
    """Routed tokens evaluated token by token, independent of the packed layout.

    The check the reference's benchmark harness runs on every forward
    (``layer.py:200-214``), with the same policy: fp32 router logits plus bias,
    top-k, softmax of the selected logits, each expert's gate/up projection,
    SwiGLU and down projection in the block's dtype (torch's own GEMMs), and the
    weighted sum in fp32 cast once. Here each expert evaluates only the
    (token, slot) pairs routed to it, gathered straight from the top-k ids, and
    adds them back by token index; no dispatch buffer, offset or permutation of
    the engine is used. Excluded from timings.
    """
    cfg = block.config
    logits = torch.nn.functional.linear(x.float(), block.router_weight) + block.routing_bias
    top = torch.topk(logits, cfg.topk, dim=-1)
    weights = torch.softmax(top.values, dim=-1)
    total = torch.zeros(x.shape, device=x.device, dtype=torch.float32)
    for expert in range(cfg.experts):
        tokens, slots = torch.nonzero(top.indices == expert, as_tuple=True)
        if tokens.numel() == 0:
            continue
        rows = x.index_select(0, tokens)
        hidden_state = swiglu_reference(torch.nn.functional.linear(rows, block.gate_up_weight[expert]))
        y = torch.nn.functional.linear(hidden_state, block.down_weight[expert]).float()
        total.index_add_(0, tokens, y * weights[tokens, slots].unsqueeze(1))
    return total.to(x.dtype)
