"""GPU parity of the draft side of a speculative round against the oracle.

* ``draft_sample``: one launch draws every row's proposal; token ids must equal
  the oracle's ``race_argmax(logits_to_probs(z_b, T), E_b)`` (the reference's
  ``sample_token``) for B = 32 rows of V = 151,936 at T = 1 and T = 0.7, and
  the first-index argmax when greedy. The kernel races log2 keys with a bound
  of their rounding and re-races near ties with torch's arithmetic; a draw
  still within a few ulp of another key is flagged (``FLAG_DRAW_BAND``), and
  every row that differs from the oracle must be flagged. Large-magnitude
  logits (|z / T| up to ~100) with crafted top-two gaps of 1e-6 to 1e-5 must
  match (gaps of 3e-6 and more unflagged); crafted exact ties (equal logits and
  equal noise) must take the lowest index.
* the draws' row statistics (max, sum exp(x - max)) against torch's, and the
  verify step fed with them equal to the verify step that computes its own.
* ``draft_sample_with_generator`` consumes a live generator exactly as the
  reference's per-row loop (engine/spec_scheduler.py:246-251) does: same tokens,
  same generator state afterwards.
* ``DraftLoop`` captured as one HIP graph (gamma = 4 steps x 2 layers, batch 16):
  proposals, every decode-attention output and the pool (tables, lengths, free
  list, stored K/V) equal the oracle's after the loop; the graph is replayed
  three times with eager work between, every replay checked.
"""

from __future__ import annotations

import pytest
import torch

from engine.attention import gather_ctx
from engine.config import SamplingConfig
from engine.kv import PagedKVCache
from engine.spec_scheduler import DraftLoop, draft_sample, draft_sample_with_generator
from oracle import attention as ref_attn
from oracle import kv_pool as ref
from oracle import sampler as S

pytestmark = pytest.mark.gpu


def _rows(seed, B, V, sigma=2.0):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(B, V, generator=g) * sigma
    e = torch.empty(B, V).exponential_(1, generator=g)
    return z, e


def _min_gap(z, e, T):
    q = S.logits_to_probs(z, T)
    top = torch.topk(q / e, 2, dim=-1).values
    return float(((top[:, 0] - top[:, 1]) / top[:, 0]).min())


def _draw(z, T, e, dev):
    B = z.shape[0]
    flags = torch.empty(B, dtype=torch.int32, device=dev)
    stats = torch.empty(B, 2, dtype=torch.float32, device=dev)
    got = draft_sample(z.to(dev), T, e.to(dev) if T > 0 else None, stats=stats, flags=flags)
    return got.tolist(), flags.tolist(), stats.cpu()


@pytest.mark.parametrize("T", [1.0, 0.7, 0.0])
def test_draft_sample_matches_the_reference_draw(cuda, T):
    B, V = 32, 151936
    z, e = _rows(60 + int(10 * T), B, V)
    want = [S.race_argmax(S.logits_to_probs(z[b], T), e[b]) for b in range(B)]
    if T > 0:
        print("draft race: min top-2 gap {:.3e}".format(_min_gap(z, e, T)))
    got, flags, stats = _draw(z, T, e, cuda)
    for b in range(B):
        assert got[b] == want[b] or flags[b], (b, got[b], want[b])
    print("{} of {} draws flagged".format(sum(1 for f in flags if f), B))
    assert sum(1 for f in flags if f) <= 1
    if T > 0:
        x = z / T
        m = x.max(-1).values
        assert torch.equal(stats[:, 0], m)
        assert torch.allclose(stats[:, 1], torch.exp(x - m[:, None]).sum(-1), rtol=2e-6)
    else:
        assert stats[:, 1].view(torch.int32).tolist() == got


@pytest.mark.parametrize("T", [0.1, 0.3])
def test_large_magnitude_logits_with_crafted_gaps(cuda, T):
    """|z / T| of 30-100: rows whose two best keys (token a, then c) are
    placed a relative gap apart by their Exp(1) entries, the leader either
    side. Keys of such logits carry rounding far above 1e-6 in the fast race,
    so these rows take the exact re-race; the tokens must be the oracle's."""
    B, V = 16, 151936
    z, e = _rows(300 + int(T * 10), B, V, sigma=3.0)
    gaps = [1e-6, 2e-6, 3e-6, 5e-6, 1e-5, 2e-5, 5e-5, 1e-4]
    for b in range(B):
        x = z[b] / T
        top = torch.topk(x, 2).indices.tolist()
        a, c = min(top), max(top)
        gap = gaps[b % len(gaps)] * (1 if b < len(gaps) else -1)
        # a small E_a lifts the pair far above every other key;
        # key_c / key_a = exp(x_c - x_a) E_a / E_c = 1 - gap
        e[b, a] = 1e-4
        e[b, c] = float(1e-4 * torch.exp((x[c] - x[a]).double()) / (1.0 - gap))
    q = S.logits_to_probs(z, T)
    want = [S.race_argmax(q[b], e[b]) for b in range(B)]
    keys = [(float(q[b, a] / e[b, a]), float(q[b, c] / e[b, c])) for b, (a, c) in
            enumerate([sorted(torch.topk(z[b] / T, 2).indices.tolist()) for b in range(B)])]
    got, flags, _ = _draw(z, T, e, cuda)
    for b in range(B):
        g = abs(gaps[b % len(gaps)])
        assert got[b] == want[b] or flags[b], (b, g, got[b], want[b], keys[b])
        if g >= 3e-6:
            assert flags[b] == 0 and got[b] == want[b], (b, g)
    print("max |z/T| {:.1f}; flagged gaps {}".format(float((z / T).abs().max()),
                                                      [gaps[b % len(gaps)] for b in range(B) if flags[b]]))


@pytest.mark.parametrize("T", [1.0, 0.7, 0.0])
def test_draft_statistics_feed_the_verify_step(cuda, T):
    """The verify step given the draft draws' row statistics decides and draws
    exactly as the one that computes the draft rows' statistics itself, and as
    the oracle (unflagged sequences)."""
    from engine import spec_scheduler as es

    B, gamma, V = 16, 4, 151936
    g = torch.Generator().manual_seed(71 + int(T * 10))
    target = torch.randn(B, gamma + 1, V, generator=g) * 2.0
    draft = target[:, :gamma] + torch.randn(B, gamma, V, generator=g)
    u = torch.rand(B, gamma, generator=g)
    noise = torch.empty(B, V).exponential_(1, generator=g)
    dnoise = torch.empty(gamma, B, V).exponential_(1, generator=g)
    d_dev = draft.to(cuda)
    props = torch.empty(B, gamma, dtype=torch.int32, device=cuda)
    stats = torch.empty(B, gamma, 2, dtype=torch.float32, device=cuda)
    for s_ in range(gamma):
        draft_sample(d_dev[:, s_], T, dnoise[s_].to(cuda) if T > 0 else None, out=props[:, s_], stats=stats[:, s_])
    x = props.cpu()
    want = S.verify_from_logits(target, draft, x, u, noise, T)
    args = (target.to(cuda), d_dev, props, u.to(cuda), noise.to(cuda) if T > 0 else None, T)
    with_stats = es.verify_sample(*args, draft_stats=stats)
    own = es.verify_sample(*args)
    fl = [a | b for a, b in zip(with_stats.flags.tolist(), own.flags.tolist())]
    for b, (w, o, r, f) in enumerate(zip(with_stats.accepted_lists(), own.accepted_lists(), want, fl)):
        assert (w == o == r) or f, (b, w, o, r)
    print("{} of {} sequences flagged".format(sum(1 for f in fl if f), B))


@pytest.mark.parametrize("V", [1000, 4097, 40000])
def test_draft_sample_odd_vocabularies_and_strided_rows(cuda, V):
    # element-wise paths (V % 4 != 0), one chunk or several, and rows that are
    # one position of a (B, gamma, V) tensor
    B, gamma = 9, 3
    g = torch.Generator().manual_seed(V)
    z3 = torch.randn(B, gamma, V, generator=g) * 2
    e = torch.empty(B, V).exponential_(1, generator=g)
    for s in range(gamma):
        want = [S.race_argmax(S.logits_to_probs(z3[b, s], 1.0), e[b]) for b in range(B)]
        got = draft_sample(z3.to(cuda)[:, s], 1.0, e.to(cuda))
        assert got.tolist() == want, s


def test_exact_ties_take_the_lowest_index(cuda):
    B, V = 4, 151936
    z, e = _rows(7, B, V)
    pairs = [(5, 150000), (100, 101), (77000, 77001), (0, 151935)]
    for b, (a, c) in enumerate(pairs):
        z[b, a] = z[b, c] = 40.0  # the two largest probabilities, equal
        e[b, a] = e[b, c] = 0.5
    want = [S.race_argmax(S.logits_to_probs(z[b], 1.0), e[b]) for b in range(B)]
    assert want == [a for a, _ in pairs]
    assert draft_sample(z.to(cuda), 1.0, e.to(cuda)).tolist() == want
    # greedy: equal maxima, the first index
    assert draft_sample(z.to(cuda), 0.0).tolist() == [a for a, _ in pairs]


def test_generator_draws_follow_the_reference_loop(cuda):
    B, V = 6, 5000
    z, _ = _rows(8, B, V)
    for T in (1.0, 0.0):
        sampling = SamplingConfig(temperature=T)
        g_ref = torch.Generator().manual_seed(99)
        g_gpu = torch.Generator().manual_seed(99)
        want = [S.sample_token(S.logits_to_probs(z[b], T), g_ref) for b in range(B)]
        got = draft_sample_with_generator(z.to(cuda), sampling, g_gpu)
        assert got == want
        assert torch.equal(g_ref.get_state(), g_gpu.get_state())


def _draft_inputs(B, gamma, layers, Hq, Hkv, d, V, seed):
    g = torch.Generator().manual_seed(seed)
    q = [[torch.randn(B, 1, Hq, d, generator=g).to(torch.bfloat16) for _ in range(layers)] for _ in range(gamma)]
    k = [[torch.randn(B, 1, Hkv, d, generator=g).to(torch.bfloat16) for _ in range(layers)] for _ in range(gamma)]
    v = [[torch.randn(B, 1, Hkv, d, generator=g).to(torch.bfloat16) for _ in range(layers)] for _ in range(gamma)]
    logits = [torch.randn(B, V, generator=g) * 2 for _ in range(gamma)]
    noise = [torch.empty(B, V).exponential_(1, generator=g) for _ in range(gamma)]
    return q, k, v, logits, noise


def test_draft_loop_as_one_graph_matches_the_oracle(cuda):
    B, gamma, layers, Hq, Hkv, d, bs, V = 16, 4, 2, 14, 2, 64, 16, 8000
    g = torch.Generator().manual_seed(3)
    ctx = torch.randint(1, 300, (B,), generator=g).tolist()
    cap = sum(-(-(L + gamma) // bs) for L in ctx) + 40
    gpu = PagedKVCache(layers, Hkv, d, cap, bs, cuda, torch.bfloat16, max_seqs=B,
                       max_blocks_per_seq=-(-(max(ctx) + gamma) // bs) + 1)
    cpu = ref.PagedKVCache(layers, Hkv, d, cap, bs, dtype=torch.bfloat16)
    for s, L in enumerate(ctx):  # the draft prompt caches
        gpu.add_sequence(s)
        cpu.add_sequence(s)
        for layer in range(layers):
            kk = torch.randn(1, L, Hkv, d, generator=g).to(torch.bfloat16)
            vv = torch.randn(1, L, Hkv, d, generator=g).to(torch.bfloat16)
            gpu.write_block(layer, [s], [0], kk.to(cuda), vv.to(cuda))
            cpu.write_block(layer, [s], [0], kk, vv)
    q, k, v, logits, noise = _draft_inputs(B, gamma, layers, Hq, Hkv, d, V, seed=4)
    # oracle: the reference's order, step by step
    want_tok = [[0] * gamma for _ in range(B)]
    want_out = []
    sids = list(range(B))
    for s in range(gamma):
        pos = [L + s for L in ctx]
        outs = []
        for layer in range(layers):
            cpu.write_block(layer, sids, pos, k[s][layer], v[s][layer])
            f32 = ref.PagedKVCache(layers, Hkv, d, cap, bs, dtype=torch.float32)
            f32.load_state(cpu.block_tables, cpu.seq_lengths, cpu.allocator.free_list)
            f32.k, f32.v = cpu.k.float(), cpu.v.float()
            outs.append(ref_attn.paged_attention_extend(q[s][layer].float(), f32, layer, sids, pos, Hq))
        want_out.append(outs)
        for b in range(B):
            want_tok[b][s] = S.race_argmax(S.logits_to_probs(logits[s][b], 1.0), noise[s][b])
    # device: the whole loop captured once
    dev = lambda xs: [[x.to(cuda) for x in row] for row in xs]  # noqa: E731
    qd, kd, vd = dev(q), dev(k), dev(v)
    ld = [x.to(cuda) for x in logits]
    nd = [x.to(cuda) for x in noise]
    sid_t = torch.arange(B, dtype=torch.int32, device=cuda)
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=cuda)
    loop = DraftLoop(gpu, gamma, 1.0)
    props = torch.empty((B, gamma), dtype=torch.int32, device=cuda)
    attn = [[torch.empty(B, 1, Hq, d, dtype=torch.bfloat16, device=cuda) for _ in range(layers)]
            for _ in range(gamma)]
    state0 = (gpu.block_tables, gpu.seq_lengths, gpu.allocator.free_list())
    # warm-up on a side stream allocates the workspaces; the eager run must
    # leave the pool as the oracle's first pass does, so snapshot / restore
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        loop.run(sid_t, ctx_t, max(ctx), qd, kd, vd, ld, nd, proposals=props, attn_out=attn)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert props.cpu().tolist() == want_tok
    assert gpu.block_tables == cpu.block_tables and gpu.seq_lengths == cpu.seq_lengths
    assert gpu.allocator.free_list() == cpu.allocator.free_list
    assert state0[0] != gpu.block_tables or state0[1] != gpu.seq_lengths
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        loop.run(sid_t, ctx_t, max(ctx), qd, kd, vd, ld, nd, proposals=props, attn_out=attn)
    for rep in range(3):
        props.fill_(-1)
        for row in attn:
            for o in row:
                o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()  # the blocks exist: the replay rewrites the same positions
        torch.cuda.synchronize()
        assert props.cpu().tolist() == want_tok, rep
        for s in range(gamma):
            for layer in range(layers):
                got, want = attn[s][layer].float().cpu(), want_out[s][layer]
                rel = float((got - want).norm() / want.norm())
                assert rel <= 2e-3, (rep, s, layer, rel)
        assert gpu.block_tables == cpu.block_tables and gpu.seq_lengths == cpu.seq_lengths
        assert gpu.allocator.free_list() == cpu.allocator.free_list
        for b in range(B):  # stored K/V of the draft tokens
            n = ctx[b] + gamma
            pair = gather_ctx(gpu, 1, b, n).cpu()
            cpair = ref_attn.gather_ctx(cpu, 1, b, n)
            assert torch.equal(pair, cpair), (rep, b)
        _ = torch.randn(64, device=cuda).sum().item()  # eager work between replays
