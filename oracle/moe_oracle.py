"""CPU oracle for the MoE feed-forward hot path. TEST INFRASTRUCTURE ONLY.

This module is a numpy restatement of the reference algorithm
(AarushRathore1729/cuda-moe-engine, package ``moe_dispatch``) used as the parity
checker for the HIP kernels. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it. The product path never calls
it and has no CPU fallback.

Conventions
-----------
* bf16 tensors are carried as float32 arrays holding bf16-representable values
  (``bf16_round``) or as raw ``uint16`` bit patterns (``bf16_bits``).
* Integer and index work (top-k ids, counts, offsets, slots, inverse map, packed
  rows) is exact; parity against it is bit-exact.
* Floating point work rounds to bf16 at the same points as the kernels and the
  reference pipeline: projection (GEMM output), activation, expert output and
  final output (reference ``experts.py:38-41``, ``_triton_gemm.py:66-70``,
  ``csrc/dispatch.cu:89-90,291``).
* Canonical slot order: the reference assigns within-expert slots with
  ``atomicAdd`` (``csrc/dispatch.cu:19-20``) and documents the order as free
  (``docs/design.md:12``). The oracle fixes it to the stable counting-sort
  order: by expert, then by flat assignment index ``p = t*K + k``.

Pinning (what checks each function; see tests/test_oracle.py)
---------------------------------------------------------------
* ``bf16_round``/``bf16_bits``: torch's ``Tensor.to(torch.bfloat16)`` on random
  and special values (ties, subnormals, inf, nan), bit for bit.
* ``topk_route``: ``torch.topk`` on tie-free inputs (exact ids), a pure-Python
  brute force ``sorted((-v, i))`` with deliberate ties, the reference KAT
  (all-zero logits, E=64 -> ids [0,1], weights exactly 0.5), and
  ``torch.softmax`` of the selected values (2e-6).
* ``dispatch_layout``: ``np.bincount``, the aligned-offset closed form,
  ``torch.sort(stable=True)``, a pure-Python counting sort on tiny inputs and
  every invariant of the reference's ``validate_case``.
* ``pack``/``combine``: ``index_select`` identities and torch's fp32
  ``(y * w).sum(1)`` (bit-exact for K <= 2).
* ``exp_f32``/``silu_f32``/``swiglu``: float64 ``exp`` (within 2 ulp over the
  whole domain), torch ``F.silu`` in fp32 then one bf16 cast (reference
  ``experts.py:38-41``).
* ``grouped_gemm``: a per-expert ``torch.matmul`` in float64 ("exact" order,
  and the "mfma" order within the fp32 error bound of it); the "mfma" order
  against a pure-Python loop over k-groups on tiny inputs; on the GPU the
  kernels match the "mfma" order in >99.99% of bf16 outputs (the rest one
  bf16 step away).
* ``block_forward``: the restated ``token_major_oracle`` (dense, token-major,
  independent of the permutation).
* ``mfma_gemm.c`` (``oracle/_build/libmoe_oracle.so``, built by
  ``__graft_entry__.build()``): the "mfma" order in C, used by ``grouped_gemm``
  for float32 inputs when the library is present; equal to the numpy form bit
  for bit (``tests/test_oracle.py``), so whole expert spans of the benchmark
  shapes can be checked in seconds.
"""

from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np

_C_LIBRARY = Path(__file__).resolve().parent / "_build" / "libmoe_oracle.so"


def build_c_checker(force: bool = False) -> Path:
    """Compile ``mfma_gemm.c`` into ``_build/libmoe_oracle.so`` with gcc (a checker, not product code)."""
    import subprocess

    if force or not _C_LIBRARY.is_file():
        _C_LIBRARY.parent.mkdir(exist_ok=True)
        tmp = _C_LIBRARY.with_suffix(".so.tmp")
        subprocess.run(["gcc", "-O3", "-fopenmp", "-mavx2", "-mfma", "-ffp-contract=off", "-shared", "-fPIC",
                        str(_C_LIBRARY.parent.parent / "mfma_gemm.c"), "-o", str(tmp)], check=True)
        tmp.replace(_C_LIBRARY)
    return _C_LIBRARY


def _load_c_gemm():
    """The C form of the "mfma" order, or None when it was not built."""
    if not _C_LIBRARY.is_file():
        return None
    try:
        lib = ctypes.CDLL(str(_C_LIBRARY))
    except OSError:
        return None
    fn = lib.moe_oracle_mfma_gemm
    fn.restype = None
    fn.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 4
    return fn


_C_GEMM = _load_c_gemm()

__all__ = [
    "bf16_bits",
    "bf16_from_bits",
    "bf16_round",
    "capacity_rows",
    "aligned_spans",
    "topk_route",
    "router_logits",
    "dispatch_layout",
    "pack",
    "combine",
    "swiglu",
    "grouped_gemm",
    "exp_f32",
    "silu_f32",
    "block_forward",
    "token_major_forward",
    "zipf_bias",
]


# ----------------------------------------------------------------------------
# bf16 helpers
# ----------------------------------------------------------------------------


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 (round-to-nearest-even) and return uint16 bits.

    NaN inputs map to a quiet NaN with the sign kept; infinities are preserved.
    """
    f = np.ascontiguousarray(values, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounding_bias = ((u >> 16) & 1) + 0x7FFF
    rounded = ((u + rounding_bias) >> 16).astype(np.uint32)
    nan = np.isnan(f)
    if nan.any():
        rounded = np.where(nan, ((u >> 16).astype(np.uint32) | 0x0040), rounded)
    return rounded.astype(np.uint16)


def bf16_from_bits(bits: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to float32 exactly."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_round(values: np.ndarray) -> np.ndarray:
    """Round to the nearest bf16 value, returned as float32."""
    return bf16_from_bits(bf16_bits(values))


def _round_to(values: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to the storage dtype ("bf16", "f16" or "f32")."""
    values = np.asarray(values, dtype=np.float32)
    if dtype == "bf16":
        return bf16_round(values)
    if dtype == "f16":
        return values.astype(np.float16).astype(np.float32)
    if dtype == "f32":
        return values
    raise ValueError(f"unknown dtype {dtype}")


# ----------------------------------------------------------------------------
# Capacity / layout formulas
# ----------------------------------------------------------------------------


def capacity_rows(tokens: int, experts: int, topk: int, alignment: int) -> int:
    """Fixed packed-row capacity (reference ``workspace.py:29-34``, ``docs/design.md:20-24``).

    Compact layout (alignment 1) uses exactly ``T*K`` rows; aligned layouts use
    ``ceil((T*K + E*(a-1) + 1)/a)*a`` so the last dynamic offset stays below
    the physical row count.
    """
    n = tokens * topk
    if alignment == 1:
        return n
    return (n + experts * (alignment - 1) + 1 + alignment - 1) // alignment * alignment


def aligned_spans(counts: np.ndarray, alignment: int) -> np.ndarray:
    """Per-expert span ``ceil(count/a)*a`` (reference ``csrc/dispatch.cu:194-205``)."""
    counts = np.asarray(counts, dtype=np.int64)
    return (counts + alignment - 1) // alignment * alignment


# ----------------------------------------------------------------------------
# Routing
# ----------------------------------------------------------------------------


def router_logits(x: np.ndarray, router_w: np.ndarray) -> np.ndarray:
    """fp32 router logits ``x.float() @ W_r^T`` (reference ``layer.py:123``).

    Accumulates in float64 and rounds once to float32, i.e. the correctly
    rounded value that any fp32 summation order approximates.
    """
    x64 = np.asarray(x, dtype=np.float64)
    w64 = np.asarray(router_w, dtype=np.float64)
    return (x64 @ w64.T).astype(np.float32)


def topk_route(logits: np.ndarray, bias: np.ndarray, topk: int):
    """Bias + top-k + selected-score softmax (reference ``csrc/dispatch.cu:325-376``).

    * ``v = logits + bias`` in fp32.
    * Top-k by value; ties resolve to the lower expert index
      (``csrc/dispatch.cu:331-333``, ``docs/design.md:16-17``).
    * Weights: ``K == 1`` -> 1.0; ``K == 2`` -> the reference closed form
      ``w0 = 1/(1+exp(v1-v0))``, ``w1 = exp(v1-v0)*w0`` (``csrc/dispatch.cu:366-374``);
      ``K > 2`` (the generalisation this build adds) -> ``exp(v_j - v_0) / sum_i exp(v_i - v_0)``
      with the sum taken in selection order.

    Returns ``(ids int32 [T,K], weights float32 [T,K], values float32 [T,K])``.
    """
    logits = np.asarray(logits, dtype=np.float32)
    bias = np.asarray(bias, dtype=np.float32)
    tokens, experts = logits.shape
    if not 1 <= topk <= experts:
        raise ValueError("topk must be in 1..experts")
    v = (logits + bias[None, :]).astype(np.float32)
    # Stable sort of -v keeps lower indices first among equal values.
    order = np.argsort(-v, axis=1, kind="stable")[:, :topk]
    ids = order.astype(np.int32)
    values = np.take_along_axis(v, order, axis=1).astype(np.float32)
    weights = np.empty((tokens, topk), dtype=np.float32)
    if topk == 1:
        weights[:] = 1.0
    elif topk == 2:
        with np.errstate(over="ignore"):
            relative = np.exp((values[:, 1] - values[:, 0]).astype(np.float32)).astype(np.float32)
        norm = (np.float32(1.0) / (np.float32(1.0) + relative)).astype(np.float32)
        weights[:, 0] = norm
        weights[:, 1] = (relative * norm).astype(np.float32)
    else:
        rel = np.exp((values - values[:, :1]).astype(np.float32)).astype(np.float32)
        total = np.zeros(tokens, dtype=np.float32)
        for j in range(topk):
            total = (total + rel[:, j]).astype(np.float32)
        inv = (np.float32(1.0) / total).astype(np.float32)
        weights[:] = (rel * inv[:, None]).astype(np.float32)
    return ids, weights, values


# ----------------------------------------------------------------------------
# Dispatch
# ----------------------------------------------------------------------------


def dispatch_layout(ids: np.ndarray, experts: int, alignment: int = 1):
    """Counts, offsets, canonical slots and inverse map of a dispatch.

    Follows reference ``csrc/dispatch.cu:13-34`` (count + compact scan),
    ``:194-205`` (aligned scan) and ``:57-74`` (``inverse[p] = offsets[e] + slot``),
    with the canonical stable slot order
    ``slot(p) = #{p' < p : ids[p'] == ids[p]}``.
    Out-of-range ids are masked as in the reference (``:19-20``): slot -1, not
    counted, inverse left as -1 here (the kernels leave it untouched).

    Returns a dict with ``counts [E]``, ``offsets [E+1]`` (int32), ``slots [N]``,
    ``inverse [T,K]`` (int32) and ``order`` (assignment indices in packed order).
    """
    ids = np.asarray(ids)
    tokens, topk = ids.shape
    flat = ids.reshape(-1).astype(np.int64)
    valid = (flat >= 0) & (flat < experts)
    counts = np.bincount(flat[valid], minlength=experts).astype(np.int64)
    spans = counts if alignment == 1 else aligned_spans(counts, alignment)
    offsets = np.zeros(experts + 1, dtype=np.int64)
    np.cumsum(spans, out=offsets[1:])
    unpadded = np.zeros(experts + 1, dtype=np.int64)
    np.cumsum(counts, out=unpadded[1:])
    keys = np.where(valid, flat, experts)  # invalid ids sort last and are dropped
    order = np.argsort(keys, kind="stable")[: int(valid.sum())]
    slots = np.full(flat.shape, -1, dtype=np.int64)
    position = np.arange(order.size, dtype=np.int64)
    slots[order] = position - unpadded[flat[order]]
    inverse = np.full(flat.shape, -1, dtype=np.int64)
    inverse[order] = offsets[flat[order]] + slots[order]
    return {
        "counts": counts.astype(np.int32),
        "offsets": offsets.astype(np.int32),
        "slots": slots.astype(np.int32),
        "inverse": inverse.reshape(tokens, topk).astype(np.int32),
        "order": order,
    }


def pack(x: np.ndarray, layout: dict, topk: int, rows: int):
    """Packed rows (reference ``csrc/dispatch.cu:57-74,207-216``).

    ``packed[inverse[p]] = x[p // K]``; padding rows inside used spans
    (``[offsets[e]+counts[e], offsets[e+1])``) are exactly zero. Rows at or past
    ``offsets[E]`` are not written by the reference; the returned ``defined``
    mask marks the rows whose content is specified.
    """
    x = np.asarray(x)
    hidden = x.shape[1]
    packed = np.zeros((rows, hidden), dtype=x.dtype)
    order = layout["order"]
    inverse = layout["inverse"].reshape(-1)
    packed[inverse[order]] = x[order // topk]
    defined = np.zeros(rows, dtype=bool)
    defined[: int(layout["offsets"][-1])] = True
    return packed, defined


# ----------------------------------------------------------------------------
# Expert compute
# ----------------------------------------------------------------------------


def grouped_gemm(a: np.ndarray, b: np.ndarray, offsets: np.ndarray, order: str = "mfma") -> np.ndarray:
    """Grouped GEMM ``C[r] = A[r] @ B[e]^T`` for rows r of expert e, fp32 result.

    Reference ``experts.py:21-35`` with ``ENDS = offsets[1:]`` and the masked
    row groups of ``_triton_gemm.py:27-70`` (fp32 accumulation; the order of the
    fp32 additions is not specified there). Two orders:

    * ``"exact"``: float64 accumulation, one rounding to fp32 (the correctly
      rounded dot product);
    * ``"mfma"`` (default): the accumulation order of the HIP kernels, which
      apply ``v_mfma_f32_16x16x32_bf16`` (fast path) or
      ``v_mfma_f32_32x32x16_bf16`` (generic path) along k in ascending order,
      modelled as: add the exact sum of each ascending group of 8 products to
      the fp32 accumulator with one round-to-nearest-even. Measured on MI355X
      for both instructions: the grouping and rounding are right (groups of
      4, 16 or 32 are far off), but the hardware sums the 8 products with a
      limited-width internal alignment, so ~0.2-0.3% of single-instruction
      fp32 results differ by one ulp; after the bf16 output rounding ~1e-5 of
      GEMM outputs are one bf16 step away from this model, versus ~5e-4 for
      the exact dot product.

    Rows at or past ``offsets[E]`` are returned as 0 (undefined for the kernels).
    """
    if order not in ("mfma", "exact"):
        raise ValueError("order must be 'mfma' or 'exact'")
    use_c = order == "mfma" and _C_GEMM is not None and np.asarray(a).dtype == np.float32
    a64 = None if use_c else np.asarray(a, dtype=np.float64)
    out = np.zeros((np.asarray(a).shape[0], b.shape[1]), dtype=np.float32)
    offsets = np.asarray(offsets, dtype=np.int64)
    for e in range(b.shape[0]):
        s, t = int(offsets[e]), int(offsets[e + 1])
        if t <= s:
            continue
        if use_c and np.asarray(b[e]).dtype == np.float32:
            out[s:t] = mfma_order_matmul_c(np.asarray(a)[s:t], np.asarray(b[e]))
            continue
        if a64 is None:
            a64 = np.asarray(a, dtype=np.float64)
        be = np.asarray(b[e], dtype=np.float64)
        if order == "exact":
            out[s:t] = (a64[s:t] @ be.T).astype(np.float32)
        else:
            out[s:t] = _mfma_order_matmul(a64[s:t], be)
    return out


def mfma_order_matmul_c(a32: np.ndarray, b32: np.ndarray, group: int = 8) -> np.ndarray:
    """``a @ b.T`` in the "mfma" order by the C checker (float32 inputs holding bf16 values)."""
    if _C_GEMM is None:
        raise RuntimeError(f"{_C_LIBRARY} is not built")
    a32 = np.ascontiguousarray(a32, dtype=np.float32)
    b32 = np.ascontiguousarray(b32, dtype=np.float32)
    m, k = a32.shape
    n = b32.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    _C_GEMM(a32.ctypes.data, b32.ctypes.data, out.ctypes.data, m, n, k, group)
    return out


def _mfma_order_matmul(a64: np.ndarray, b64: np.ndarray, group: int = 8) -> np.ndarray:
    """``a @ b.T`` accumulated as: acc = fp32(acc + exact sum of k-group), groups ascending."""
    m, k = a64.shape
    n = b64.shape[0]
    pad = (-k) % group
    if pad:
        a64 = np.pad(a64, ((0, 0), (0, pad)))
        b64 = np.pad(b64, ((0, 0), (0, pad)))
    groups = a64.shape[1] // group
    ag = a64.reshape(m, groups, group).transpose(1, 0, 2)  # [G, m, 8]
    bg = b64.reshape(n, groups, group).transpose(1, 2, 0)  # [G, 8, n]
    acc = np.zeros((m, n), dtype=np.float32)
    col_block = max(1, (1 << 24) // max(1, m * 64))
    for c0 in range(0, n, col_block):
        c1 = min(n, c0 + col_block)
        part = np.zeros((m, c1 - c0), dtype=np.float32)
        for g0 in range(0, groups, 64):
            sums = np.matmul(ag[g0:g0 + 64], bg[g0:g0 + 64, :, c0:c1])  # exact group sums
            for i in range(sums.shape[0]):
                part = (part.astype(np.float64) + sums[i]).astype(np.float32)
        acc[:, c0:c1] = part
    return acc


# exp for SiLU, reproducible bit for bit on the GPU: Cody-Waite range
# reduction x = n*ln2 + r (ln2 split into a 16-bit head and a tail so n*ln2_hi is
# exact), then the degree-7 Taylor polynomial of e^r in Horner form, every step
# a separately rounded fp32 operation (no fused multiply-add), then 2^n scaling.
# |r| <= ln2/2 gives a truncation error below 1e-8 relative; the result is
# within 2 ulp of exp (checked against float64 exp in tests/test_oracle.py).
EXP_LOG2E = np.float32(1.4426950216293335)        # 0x3fb8aa3b
EXP_LN2_HI = np.float32(0.693145751953125)        # 0x3f317200
EXP_LN2_LO = np.float32(1.428606765330187e-06)    # 0x35bfbe8e
EXP_TAYLOR = tuple(np.float32(1.0 / math.factorial(k)) for k in range(7, -1, -1))
EXP_MAX = np.float32(88.0)     # above: +inf
EXP_MIN = np.float32(-80.0)    # below: 0 (1 + e^x rounds to 1 anyway)


def exp_f32(x: np.ndarray) -> np.ndarray:
    """fp32 exp with the kernels' exact operation sequence."""
    x = np.asarray(x, dtype=np.float32)
    n = np.rint((x * EXP_LOG2E).astype(np.float32)).astype(np.float32)
    r = (x - (n * EXP_LN2_HI).astype(np.float32)).astype(np.float32)
    r = (r - (n * EXP_LN2_LO).astype(np.float32)).astype(np.float32)
    p = np.full_like(r, EXP_TAYLOR[0])
    for c in EXP_TAYLOR[1:]:
        p = ((p * r).astype(np.float32) + c).astype(np.float32)
    with np.errstate(invalid="ignore"):
        ni = np.where(np.isfinite(n), n, 0).astype(np.int32)
    out = np.ldexp(p, ni).astype(np.float32)
    out = np.where(x > EXP_MAX, np.float32(np.inf), out)
    out = np.where(x < EXP_MIN, np.float32(0.0), out)
    return np.where(np.isnan(x), x, out).astype(np.float32)


def silu_f32(g: np.ndarray) -> np.ndarray:
    """``g / (1 + exp(-g))`` in fp32 (reference ``csrc/dispatch.cu:288-291``), exp as ``exp_f32``."""
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        return (g / (np.float32(1.0) + exp_f32(-g))).astype(np.float32)


def swiglu(projection: np.ndarray, valid_rows: int, dtype: str = "bf16") -> np.ndarray:
    """SwiGLU of a ``[R, 2I]`` projection (reference ``csrc/dispatch.cu:277-292``).

    ``act = round(silu(g) * u)`` in fp32 with one cast; rows ``>= valid_rows``
    are exactly zero.
    """
    projection = np.asarray(projection, dtype=np.float32)
    width = projection.shape[1] // 2
    gate, up = projection[:, :width], projection[:, width:]
    act = _round_to((silu_f32(gate) * up).astype(np.float32), dtype)
    act[valid_rows:] = 0.0
    return act


def combine(expert_output: np.ndarray, inverse: np.ndarray, weights: np.ndarray,
            dtype: str = "bf16") -> np.ndarray:
    """Weighted gather-reduce (reference ``csrc/dispatch.cu:76-93``).

    ``out[t] = round(sum_k w[t,k] * y[inverse[t,k]])`` with fp32 products and a
    fp32 running sum taken in k order without fused multiply-add; rows whose
    inverse is outside ``[0, R)`` are skipped.
    """
    y = np.asarray(expert_output, dtype=np.float32)
    inverse = np.asarray(inverse, dtype=np.int64)
    weights = np.asarray(weights, dtype=np.float32)
    tokens, topk = inverse.shape
    rows, hidden = y.shape
    total = np.zeros((tokens, hidden), dtype=np.float32)
    for k in range(topk):
        row = inverse[:, k]
        ok = (row >= 0) & (row < rows)
        term = np.zeros((tokens, hidden), dtype=np.float32)
        term[ok] = (y[row[ok]] * weights[ok, k][:, None]).astype(np.float32)
        total = (total + term).astype(np.float32)
    return _round_to(total, dtype)


# ----------------------------------------------------------------------------
# Whole block
# ----------------------------------------------------------------------------


def block_forward(x, router_w, bias, gate_up, down, topk, alignment=8, ids=None,
                  weights=None, gemm_order="mfma"):
    """Expert-major block forward with the kernels' rounding points.

    Restates ``MoEBlock.forward`` for ``implementation="cuda_fused"``
    (reference ``layer.py:122-197``): route -> aligned dispatch -> gate/up GEMM
    (bf16 projection) -> SwiGLU (bf16) -> down GEMM (bf16) -> combine (bf16).

    ``x`` holds bf16 values (float32 array). ``ids``/``weights`` may be given to
    evaluate the downstream stages on a fixed routing. ``gemm_order`` selects
    the fp32 accumulation order of the GEMMs (see ``grouped_gemm``). Returns a
    dict of every intermediate.
    """
    x = np.asarray(x, dtype=np.float32)
    tokens, hidden = x.shape
    experts, two_i, _ = gate_up.shape
    logits = router_logits(x, router_w)
    if ids is None:
        ids, weights, _ = topk_route(logits, bias, topk)
    layout = dispatch_layout(ids, experts, alignment)
    rows = capacity_rows(tokens, experts, topk, alignment)
    packed, _ = pack(x, layout, topk, rows)
    offsets = layout["offsets"]
    projection = bf16_round(grouped_gemm(packed, gate_up, offsets, order=gemm_order))
    activated = swiglu(projection, int(offsets[-1]))
    expert_output = bf16_round(grouped_gemm(activated, down, offsets, order=gemm_order))
    output = combine(expert_output, layout["inverse"], weights)
    return {
        "logits": logits,
        "ids": ids,
        "weights": weights,
        "layout": layout,
        "rows": rows,
        "packed": packed,
        "projection": projection,
        "activated": activated,
        "expert_output": expert_output,
        "output": output,
    }


def token_major_forward(x, gate_up, down, ids, weights, token_index=None, order="exact"):
    """Dense token-major evaluation (reference ``layer.py:200-214``).

    Independent of dispatch: for each expert, evaluates every (selected) token
    densely and adds ``output * probability`` in fp32 in expert order, then
    rounds once. Projection, activation and expert output are rounded to bf16
    as the reference's ``F.linear`` on bf16 tensors does. ``token_index``
    restricts the evaluation to a subset of tokens (for full-size samples).
    ``order`` is the fp32 accumulation order of the dot products ("exact":
    float64 then one rounding; "mfma": see ``grouped_gemm``).
    """
    x = np.asarray(x, dtype=np.float32)
    ids = np.asarray(ids)
    weights = np.asarray(weights, dtype=np.float32)
    if token_index is not None:
        x, ids, weights = x[token_index], ids[token_index], weights[token_index]
    tokens, hidden = x.shape
    experts, two_i, _ = gate_up.shape
    width = two_i // 2
    expected = np.zeros((tokens, hidden), dtype=np.float32)
    for e in range(experts):
        probability = np.zeros(tokens, dtype=np.float32)
        for k in range(ids.shape[1]):
            probability = (probability + np.where(ids[:, k] == e, weights[:, k], 0)).astype(np.float32)
        rows = np.nonzero(probability)[0]
        if rows.size == 0:
            continue
        one = np.array([0, rows.size])
        proj = bf16_round(grouped_gemm(x[rows], np.asarray(gate_up[e])[None], one, order=order))
        act = bf16_round((silu_f32(proj[:, :width]) * proj[:, width:]).astype(np.float32))
        out = bf16_round(grouped_gemm(act, np.asarray(down[e])[None], one, order=order))
        expected[rows] = (expected[rows] + out * probability[rows, None]).astype(np.float32)
    return bf16_round(expected)


# ----------------------------------------------------------------------------
# Workload helpers
# ----------------------------------------------------------------------------


def zipf_bias(experts: int, exponent: float = 1.2, scale: float = 1.75, seed: int = 0):
    """Zipf-shaped router bias for the skewed fine-grained configuration.

    ``r`` is a seeded permutation of ``1..E``; ``p_e ~ r_e^-s``;
    ``bias_e = scale * ln(p_e / max p)``.
    """
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(np.arange(1, experts + 1)).astype(np.float64)
    p = ranks ** (-exponent)
    return (scale * np.log(p / p.max())).astype(np.float32)


def expert_flops(tokens: int, topk: int, hidden: int, intermediate: int) -> float:
    """Algorithmic expert-GEMM FLOPs: ``6*N*H*I`` over real assignments only."""
    return 6.0 * tokens * topk * hidden * intermediate


def dispatch_bytes(tokens, hidden, topk, padding_rows, elem=2):
    """Algorithmic dispatch bytes: x read once, packed rows + pad rows written, ids and inverse."""
    n = tokens * topk
    return tokens * hidden * elem + n * hidden * elem + padding_rows * hidden * elem + n * 8


def combine_bytes(tokens, hidden, topk, elem=2):
    """Algorithmic combine bytes: K rows gathered, one row written, inverse and weights read."""
    n = tokens * topk
    return n * hidden * elem + tokens * hidden * elem + n * 8


def _selfcheck():  # pragma: no cover - manual use
    ids = np.array([[1, 0], [1, 1], [0, 2]])
    lay = dispatch_layout(ids, 3, 1)
    assert lay["inverse"].tolist() == [[2, 0], [3, 4], [1, 5]], lay
    assert math.isclose(float(bf16_round(np.float32([1.00390625]))[0]), 1.0)


if __name__ == "__main__":  # pragma: no cover
    _selfcheck()
    print("ok")
