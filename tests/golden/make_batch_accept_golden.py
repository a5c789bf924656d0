"""Write golden vectors for ``batch_accept`` driven by a live CPU generator.

The reference's own tests pin ``batch_accept`` only on one-hot (greedy)
inputs, where no randomness matters. Its sampled-mode behaviour -- which
uniforms and exponential rows it draws from the generator, and in which order
-- is fixed only by running it. This script runs the reference's
``engine.spec_scheduler.batch_accept`` (from /root/reference, in the build
container only) on small seeded inputs and records inputs, outputs and the
generator's next draw (a witness of how much randomness was consumed) into
``batch_accept_golden.json`` next to this file.

Inputs follow the vocab-8 toy of the CPU check workload: p and q are softmax
rows of N(0, 1.5^2) logits, proposals drawn from q; plus a larger-vocabulary case.
"""

from __future__ import annotations

import json
import os
import sys

import torch

REFERENCE = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def _case(seed: int, batch: int, gamma: int, vocab: int, sigma: float, gen_seed: int, batch_accept):
    g = torch.Generator().manual_seed(seed)
    pl = torch.randn((batch, gamma + 1, vocab), generator=g) * sigma
    ql = torch.randn((batch, gamma, vocab), generator=g) * sigma
    p = torch.softmax(pl, dim=-1)
    q = torch.softmax(ql, dim=-1)
    props = [[int(torch.multinomial(q[b, j], 1, generator=g)) for j in range(gamma)] for b in range(batch)]
    sids = [3 * b + 1 for b in range(batch)]  # non-contiguous ids, dict order = batch order
    p_by = {s: p[b] for b, s in enumerate(sids)}
    q_by = {s: [q[b, j] for j in range(gamma)] for b, s in enumerate(sids)}
    x_by = {s: props[b] for b, s in enumerate(sids)}
    gen = torch.Generator().manual_seed(gen_seed)
    out = batch_accept(p_by, q_by, x_by, gen)
    witness = float(torch.rand(1, generator=gen).item())
    return {
        "seed": seed, "gen_seed": gen_seed, "batch": batch, "gamma": gamma, "vocab": vocab,
        "sids": sids,
        "p": p.reshape(-1).tolist(), "q": q.reshape(-1).tolist(), "proposals": props,
        "accepted": [out[s] for s in sids],
        "next_uniform": witness,
    }


def main() -> None:
    sys.path.insert(0, REFERENCE)
    from engine.spec_scheduler import batch_accept  # noqa: E402  (reference code, this container only)

    cases = []
    for i in range(6):
        cases.append(_case(100 + i, 4, 4, 8, 1.5, 7 + i, batch_accept))
    cases.append(_case(200, 2, 3, 200, 2.0, 11, batch_accept))
    cases.append(_case(201, 2, 2, 50, 0.3, 12, batch_accept))  # flat rows: mostly accepted
    path = os.path.join(HERE, "batch_accept_golden.json")
    with open(path, "w") as f:
        json.dump({"torch": torch.__version__, "cases": cases}, f)
    print(path, len(cases), "cases")


if __name__ == "__main__":
    main()
