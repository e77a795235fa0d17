"""Pins the CPU oracle before it is trusted as the parity checker.

Each oracle function is checked against something independent of its own
formula: torch library routines (bf16 cast, topk, softmax, stable sort,
bincount, matmul), pure-Python brute force on tiny inputs, the reference's
known answers (zero-logit tie KAT, capacity rows of the benchmark shapes), and
invariants of the reference's validate_case. Two mutation tests plant a
plausible mistake in a copy of an oracle function and show the checks catch it.
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import moe_oracle as oracle


# --------------------------------------------------------------------------- bf16
def test_bf16_round_matches_torch_bit_for_bit():
    rng = np.random.default_rng(0)
    values = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1e-45, 1.17549435e-38],
                 dtype=np.float32),
    ]).astype(np.float32)
    # Exact ties between two bf16 values (round half to even).
    base = rng.integers(0, 1 << 15, 2000).astype(np.uint32) << 16
    ties = (base | 0x8000).view(np.float32)
    values = np.concatenate([values, ties])
    ours = oracle.bf16_bits(values)
    theirs = torch.from_numpy(values.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = ~np.isnan(values)
    np.testing.assert_array_equal(ours[finite], theirs[finite])
    assert np.all(np.isnan(oracle.bf16_from_bits(ours[~finite])))


def test_bf16_round_trip_is_identity_on_bf16_values():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    values = oracle.bf16_from_bits(bits)
    finite = np.isfinite(values)
    np.testing.assert_array_equal(oracle.bf16_bits(values[finite]), bits[finite])


# --------------------------------------------------------------------------- routing
@pytest.mark.parametrize("experts,topk", [(1, 1), (2, 1), (2, 2), (8, 2), (16, 6), (64, 6), (64, 8), (33, 3)])
def test_topk_matches_torch_on_continuous_scores(experts, topk):
    g = torch.Generator().manual_seed(experts * 10 + topk)
    logits = torch.randn(300, experts, generator=g)
    bias = torch.randn(experts, generator=g)
    ids, weights, values = oracle.topk_route(logits.numpy(), bias.numpy(), topk)
    selected, expected = torch.topk(logits + bias, topk, dim=-1)
    np.testing.assert_array_equal(ids, expected.numpy())
    np.testing.assert_array_equal(values, selected.numpy())
    np.testing.assert_allclose(weights, torch.softmax(selected, -1).numpy(), rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("topk", [1, 2, 3, 6])
def test_topk_brute_force_with_ties(topk):
    rng = np.random.default_rng(topk)
    logits = rng.integers(0, 3, (200, 9)).astype(np.float32)
    bias = rng.integers(0, 2, 9).astype(np.float32)
    ids, _, _ = oracle.topk_route(logits, bias, topk)
    for t in range(logits.shape[0]):
        v = logits[t] + bias
        expect = sorted(range(9), key=lambda i: (-v[i], i))[:topk]
        assert list(ids[t]) == expect


def test_topk_zero_logits_known_answer():
    """Reference tests/test_gpu_router.py:27-38: zero logits, E=64 -> ids [0, 1], weights 0.5."""
    ids, weights, _ = oracle.topk_route(np.zeros((5, 64), np.float32), np.zeros(64, np.float32), 2)
    assert ids.tolist() == [[0, 1]] * 5
    assert np.all(weights == 0.5)
    ids, weights, _ = oracle.topk_route(np.zeros((0, 64), np.float32), np.zeros(64, np.float32), 2)
    assert ids.shape == (0, 2)


def test_topk2_weights_closed_form_and_sum():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((500, 8)).astype(np.float32)
    _, w, v = oracle.topk_route(logits, np.zeros(8, np.float32), 2)
    r = np.exp(np.float64(v[:, 1]) - np.float64(v[:, 0]))
    np.testing.assert_allclose(w[:, 0], 1 / (1 + r), rtol=1e-6)
    np.testing.assert_allclose(w[:, 1], r / (1 + r), rtol=1e-6)
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)


def test_router_logits_match_float64_matmul():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 256, generator=g).bfloat16().float()
    w = torch.randn(8, 256, generator=g) / 16
    got = oracle.router_logits(x.numpy(), w.numpy())
    np.testing.assert_array_equal(got, (x.double() @ w.double().T).float().numpy())


# --------------------------------------------------------------------------- dispatch
def _brute_layout(ids, experts, alignment):
    flat = [int(v) for v in ids.reshape(-1)]
    counts = [sum(1 for v in flat if v == e) for e in range(experts)]
    spans = [-(-c // alignment) * alignment for c in counts]
    offsets = [0]
    for s in spans:
        offsets.append(offsets[-1] + s)
    slots, inverse = [], []
    for p, e in enumerate(flat):
        s = sum(1 for q in range(p) if flat[q] == e)
        slots.append(s)
        inverse.append(offsets[e] + s)
    return counts, offsets, slots, inverse


@pytest.mark.parametrize("tokens,experts,topk,alignment", [
    (0, 4, 2, 1), (1, 4, 2, 8), (7, 3, 1, 1), (13, 5, 3, 8), (20, 8, 2, 16), (9, 64, 6, 8)])
def test_dispatch_layout_brute_force(tokens, experts, topk, alignment):
    rng = np.random.default_rng(tokens + experts)
    ids = rng.integers(0, experts, (tokens, topk)).astype(np.int32)
    layout = oracle.dispatch_layout(ids, experts, alignment)
    counts, offsets, slots, inverse = _brute_layout(ids, experts, alignment)
    assert layout["counts"].tolist() == counts
    assert layout["offsets"].tolist() == offsets
    assert layout["slots"].tolist() == slots
    assert layout["inverse"].reshape(-1).tolist() == inverse


@pytest.mark.parametrize("alignment", [1, 8, 16, 128])
def test_dispatch_layout_library_and_invariants(alignment):
    rng = np.random.default_rng(alignment)
    tokens, experts, topk = 1000, 16, 2
    ids = rng.integers(0, experts, (tokens, topk)).astype(np.int32)
    ids[:, 0] = np.minimum(ids[:, 0], 9)  # leave some experts lightly used
    layout = oracle.dispatch_layout(ids, experts, alignment)
    flat = ids.reshape(-1)
    np.testing.assert_array_equal(layout["counts"], np.bincount(flat, minlength=experts))
    spans = -(-np.bincount(flat, minlength=experts) // alignment) * alignment
    np.testing.assert_array_equal(np.diff(layout["offsets"]), spans)
    # Canonical order equals torch's stable sort of the flat ids.
    order = torch.sort(torch.from_numpy(flat.astype(np.int64)), stable=True).indices.numpy()
    np.testing.assert_array_equal(layout["order"], order)
    inverse = layout["inverse"].reshape(-1).astype(np.int64)
    rows = oracle.capacity_rows(tokens, experts, topk, alignment)
    if alignment == 1:
        np.testing.assert_array_equal(np.sort(inverse), np.arange(tokens * topk))
    else:
        assert np.unique(inverse).size == inverse.size and inverse.min() >= 0 and inverse.max() < rows
    owner = np.searchsorted(layout["offsets"][1:], inverse, side="right")
    np.testing.assert_array_equal(owner, flat)
    x = rng.integers(-1000, 1000, (tokens, 24)).astype(np.int16)
    packed, defined = oracle.pack(x, layout, topk, rows)
    np.testing.assert_array_equal(packed[inverse].reshape(tokens, topk, 24), np.repeat(x[:, None], topk, 1))
    occupied = np.zeros(rows, bool)
    occupied[inverse] = True
    assert np.all(packed[defined & ~occupied] == 0)


def test_dispatch_masks_out_of_range_ids():
    ids = np.array([[0, 9], [1, -1], [2, 2]], np.int32)
    layout = oracle.dispatch_layout(ids, 3, 1)
    assert layout["counts"].tolist() == [1, 1, 2]
    assert layout["slots"].tolist() == [0, -1, 0, -1, 0, 1]
    assert layout["inverse"].tolist() == [[0, -1], [1, -1], [2, 3]]


def test_capacity_rows_of_the_baseline_shapes():
    """Capacity R of the benchmark configurations (alignment 8; compact transport R = N)."""
    assert oracle.capacity_rows(128, 8, 2, 8) == 320
    assert oracle.capacity_rows(4096, 8, 2, 1) == 8192
    assert [oracle.capacity_rows(t, 16, 2, 8) for t in (256, 1024, 4096)] == [632, 2168, 8312]
    assert [oracle.capacity_rows(t, 8, 2, 8) for t in (1, 16, 4096)] == [64, 96, 8256]
    assert oracle.capacity_rows(8192, 64, 6, 8) == 49608


def test_mutation_unstable_order_is_caught():
    """Planting a wrong slot order (descending p within an expert) must fail the brute force."""
    ids = np.array([[1, 0], [1, 1], [0, 2]], np.int32)

    def mutated(ids, experts, alignment):
        layout = oracle.dispatch_layout(ids, experts, alignment)
        flat = ids.reshape(-1)
        for e in range(experts):
            members = np.nonzero(flat == e)[0]
            layout["slots"][members] = layout["slots"][members][::-1]
        return layout

    _, _, slots, _ = _brute_layout(ids, 3, 1)
    assert oracle.dispatch_layout(ids, 3, 1)["slots"].tolist() == slots
    assert mutated(ids, 3, 1)["slots"].tolist() != slots


# --------------------------------------------------------------------------- combine / swiglu / gemm
@pytest.mark.parametrize("topk", [1, 2])
def test_combine_matches_torch_fp32_sum_bit_exactly(topk):
    g = torch.Generator().manual_seed(topk)
    tokens, hidden = 77, 40
    y = torch.randn(tokens * topk, hidden, generator=g).bfloat16()
    inverse = torch.randperm(tokens * topk, generator=g).view(tokens, topk)
    w = torch.softmax(torch.randn(tokens, topk, generator=g), -1)
    expected = (y.float()[inverse] * w[:, :, None]).sum(1).bfloat16().float().numpy()
    got = oracle.combine(y.float().numpy(), inverse.numpy(), w.numpy(), "bf16")
    np.testing.assert_array_equal(got, expected)


def test_combine_sequential_order_for_larger_k():
    rng = np.random.default_rng(2)
    tokens, topk, hidden = 10, 6, 8
    y = oracle.bf16_round(rng.standard_normal((tokens * topk, hidden)).astype(np.float32))
    inverse = rng.permutation(tokens * topk).reshape(tokens, topk).astype(np.int32)
    w = rng.random((tokens, topk)).astype(np.float32)
    got = oracle.combine(y, inverse, w, "f32")
    for t in range(tokens):
        acc = np.zeros(hidden, np.float32)
        for k in range(topk):
            acc = (acc + (y[inverse[t, k]] * w[t, k]).astype(np.float32)).astype(np.float32)
        np.testing.assert_array_equal(got[t], acc)


def test_combine_skips_rows_out_of_range():
    y = np.ones((4, 3), np.float32)
    got = oracle.combine(y, np.array([[0, 4], [-1, 1]]), np.array([[0.5, 0.5], [0.25, 0.75]], np.float32), "f32")
    np.testing.assert_array_equal(got, [[0.5] * 3, [0.75] * 3])


def test_swiglu_matches_torch_silu():
    g = torch.Generator().manual_seed(4)
    proj = torch.randn(37, 34, generator=g).bfloat16()
    got = oracle.swiglu(proj.float().numpy(), 21)
    gate, up = proj.float().chunk(2, -1)
    expected = (torch.nn.functional.silu(gate) * up).bfloat16().float().numpy()
    np.testing.assert_allclose(got[:21], expected[:21], rtol=2e-2, atol=2e-2)
    assert np.mean(got[:21] == expected[:21]) > 0.97
    assert np.all(got[21:] == 0)


def test_grouped_gemm_matches_per_expert_torch_matmul():
    g = torch.Generator().manual_seed(5)
    offsets = np.array([0, 8, 8, 40, 48], np.int32)
    a = torch.randn(50, 32, generator=g)
    b = torch.randn(4, 24, 32, generator=g)
    got = oracle.grouped_gemm(a.numpy(), b.numpy(), offsets, order="exact")
    for e in range(4):
        s, t = offsets[e], offsets[e + 1]
        np.testing.assert_allclose(got[s:t], (a[s:t].double() @ b[e].double().T).float().numpy(), rtol=1e-6)
    assert np.all(got[48:] == 0)


# --------------------------------------------------------------------------- whole block
@pytest.mark.parametrize("topk,experts", [(1, 8), (2, 8), (6, 16)])
def test_block_expert_major_equals_token_major(topk, experts):
    g = torch.Generator().manual_seed(topk)
    h, i, tokens = 32, 64, 57
    x = torch.randn(tokens, h, generator=g).bfloat16().float().numpy()
    router = (torch.randn(experts, h, generator=g) / h**0.5).numpy()
    gate_up = (torch.randn(experts, 2 * i, h, generator=g) / h**0.5).bfloat16().float().numpy()
    down = (torch.randn(experts, h, i, generator=g) / i**0.5).bfloat16().float().numpy()
    bias = np.zeros(experts, np.float32)
    ref = oracle.block_forward(x, router, bias, gate_up, down, topk, 8)
    dense = oracle.token_major_forward(x, gate_up, down, ref["ids"], ref["weights"])
    diff = np.abs(ref["output"] - dense)
    assert diff.max() <= 1.6e-2
    assert np.linalg.norm(ref["output"] - dense) / np.linalg.norm(dense) <= 5e-4


def test_zipf_bias_produces_the_skewed_workload():
    """E=64, top-6, logits ~ N(0,1) + Zipf bias: >= 3 empty experts and >= 2 experts above 15%."""
    rng = np.random.default_rng(0)
    bias = oracle.zipf_bias(64, exponent=1.2, scale=1.75, seed=0)
    logits = rng.standard_normal((8192, 64)).astype(np.float32)
    ids, _, _ = oracle.topk_route(logits, bias, 6)
    counts = np.bincount(ids.reshape(-1), minlength=64)
    assert (counts == 0).sum() >= 3
    assert (counts / counts.sum() > 0.15).sum() >= 2


def test_flop_and_byte_models():
    assert oracle.expert_flops(4096, 2, 4096, 14336) == pytest.approx(2.886e12, rel=1e-3)
    assert oracle.combine_bytes(4096, 2048, 2) == pytest.approx(50.4e6, rel=2e-3)
    assert oracle.dispatch_bytes(4096, 2048, 2, 0) == pytest.approx(50.4e6, rel=2e-3)


def test_all_permutations_tiny_brute_force():
    """Every id assignment for T=2, K=2, E=3 against the brute force counting sort."""
    for combo in itertools.product(range(3), repeat=4):
        ids = np.array(combo, np.int32).reshape(2, 2)
        for alignment in (1, 2):
            layout = oracle.dispatch_layout(ids, 3, alignment)
            counts, offsets, slots, inverse = _brute_layout(ids, 3, alignment)
            assert layout["inverse"].reshape(-1).tolist() == inverse
            assert layout["offsets"].tolist() == offsets


# --------------------------------------------------------------------------- exp / MFMA order
def _ulp_error(got, ref64):
    ref32 = ref64.astype(np.float32)
    spacing = np.spacing(np.abs(ref32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref64) / spacing


def test_exp_f32_within_two_ulp_of_float64_exp():
    x = np.concatenate([np.linspace(-80, 88, 2_000_003, dtype=np.float32),
                        np.random.default_rng(0).uniform(-20, 20, 200_000).astype(np.float32)])
    got = oracle.exp_f32(x)
    err = _ulp_error(got, np.exp(x.astype(np.float64)))
    assert err.max() <= 2.0, err.max()
    assert np.mean(err <= 0.5) > 0.5


def test_exp_f32_special_values():
    x = np.array([0.0, -0.0, 88.5, 1e30, -80.5, -1e30, np.inf, -np.inf, np.nan], np.float32)
    got = oracle.exp_f32(x)
    assert got[0] == 1.0 and got[1] == 1.0
    assert np.isinf(got[2]) and np.isinf(got[3]) and np.isinf(got[6])
    assert got[4] == 0.0 and got[5] == 0.0 and got[7] == 0.0
    assert np.isnan(got[8])


def test_silu_f32_matches_torch_silu():
    g = np.random.default_rng(1).standard_normal(100_000).astype(np.float32) * 6
    got = oracle.silu_f32(g)
    ref = torch.nn.functional.silu(torch.from_numpy(g).double()).numpy()
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 4e-7


def test_mfma_order_matches_python_loop_definition():
    rng = np.random.default_rng(3)
    a = oracle.bf16_round(rng.standard_normal((3, 40)).astype(np.float32))
    b = oracle.bf16_round(rng.standard_normal((1, 5, 40)).astype(np.float32))
    got = oracle.grouped_gemm(a, b, np.array([0, 3]), order="mfma")
    for i in range(3):
        for j in range(5):
            acc = np.float32(0.0)
            for g0 in range(0, 40, 8):
                exact = sum(float(a[i, k]) * float(b[0, j, k]) for k in range(g0, g0 + 8))
                acc = np.float32(float(acc) + exact)
            assert got[i, j] == acc


def test_mfma_order_is_within_fp32_bound_of_exact():
    rng = np.random.default_rng(4)
    a = oracle.bf16_round(rng.standard_normal((64, 1024)).astype(np.float32))
    b = oracle.bf16_round((rng.standard_normal((2, 96, 1024)) / 32).astype(np.float32))
    offsets = np.array([0, 30, 64])
    mfma = oracle.grouped_gemm(a, b, offsets, order="mfma")
    exact = oracle.grouped_gemm(a, b, offsets, order="exact")
    bound = 128 * np.finfo(np.float32).eps * (np.abs(a) @ np.abs(b[0]).T).max()
    assert np.max(np.abs(mfma - exact)) <= bound
    assert np.any(mfma != exact)  # the orders do differ somewhere


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 33, 17), (40, 65, 200), (17, 96, 1030)])
def test_mfma_order_c_checker_equals_numpy_form(m, n, k):
    """The C form (used for whole expert spans) and the numpy form agree bit for bit,
    including a k that is not a whole number of groups and a wide dynamic range."""
    assert oracle._C_GEMM is not None, "oracle/_build/libmoe_oracle.so was not built"
    rng = np.random.default_rng(m * 1000 + n + k)
    scale = np.exp2(rng.integers(-12, 12, size=(1, k))).astype(np.float32)
    a = oracle.bf16_round((rng.standard_normal((m, k)) * scale).astype(np.float32))
    b = oracle.bf16_round((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))
    c = oracle.mfma_order_matmul_c(a, b)
    ref = oracle._mfma_order_matmul(a.astype(np.float64), b.astype(np.float64))
    np.testing.assert_array_equal(c, ref)
    # A different grouping is a different model: groups of 4 disagree somewhere.
    if k >= 64:
        assert not np.array_equal(oracle.mfma_order_matmul_c(a, b, group=4), c)
