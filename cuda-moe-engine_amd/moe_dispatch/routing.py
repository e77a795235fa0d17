"""Synthetic routed tokens from one seeded generator (made before any timing starts).

Restates ``make_case`` (reference ``src/moe_dispatch/routing.py:6-17``): from
one seeded generator, x ~ N(0,1) in the requested dtype, then fp32 logits
~ N(0,1) (``skewed`` adds 5 to the first K experts), top-k, softmax of the
selected logits.
"""

import torch


def make_case(tokens, hidden, experts, topk, dtype, pattern, seed, device="cuda"):
    generator = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn((tokens, hidden), device=device, dtype=dtype, generator=generator)
    logits = torch.randn((tokens, experts), device=device, generator=generator)
    if pattern == "skewed":
        logits[:, :topk] += 5.0
    elif pattern != "balanced":
        raise ValueError(f"unknown pattern: {pattern}")
    selected, ids64 = torch.topk(logits, topk, dim=-1)
    weights = torch.softmax(selected, dim=-1).contiguous()
    return x, ids64.to(torch.int32).contiguous(), ids64.contiguous(), weights


def make_transport_case(tokens, hidden, experts, topk, dtype, seed, device="cuda"):
    """Transport workload with i.i.d. uniform expert ids (duplicates within a token allowed).

    x ~ N(0,1); ids ~ randint(0, E); weights = softmax of N(0,1) logits [T,K].
    """
    generator = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn((tokens, hidden), device=device, dtype=dtype, generator=generator)
    ids64 = torch.randint(0, experts, (tokens, topk), device=device, generator=generator)
    logits = torch.randn((tokens, topk), device=device, generator=generator)
    weights = torch.softmax(logits, dim=-1).contiguous()
    return x, ids64.to(torch.int32).contiguous(), ids64.contiguous(), weights


def zipf_bias(experts, exponent=1.2, scale=1.75, seed=0):
    """Router bias of the skewed fine-grained workload (T=8192, H=2048, I=1408, E=64, top-6), fp32 ``[E]``.

    Expert e gets a Zipf weight ``p_e = r_e ** -exponent`` for a seeded random
    rank permutation ``r`` of 1..E, and ``bias_e = scale * ln(p_e / max p)``:
    0 for the top-ranked expert, increasingly negative below it. With N(0,1)
    logits and top-6 over 64 experts this leaves several experts without tokens
    and gives a few more than 15% of the assignments.
    """
    import numpy as np

    ranks = np.random.default_rng(seed).permutation(np.arange(1, experts + 1)).astype(np.float64)
    weight = ranks ** (-exponent)
    return torch.from_numpy((scale * np.log(weight / weight.max())).astype(np.float32))
