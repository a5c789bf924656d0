"""Host logic of the continuous-batching driver (no GPU): admission order,
lifetime reservation, the batch cap and the request stream."""

from __future__ import annotations

import pytest

from engine.continuous import DriverResult, Request, SpecContinuousDriver, poisson_requests


class _Alloc:
    def __init__(self, capacity):
        self.capacity = capacity
        self.num_free = capacity


class _KV:
    """Records admissions; a prompt takes ceil(len / block_size) blocks."""

    def __init__(self, capacity, block_size):
        self.block_size = block_size
        self.allocator = _Alloc(capacity)
        self.device = "cpu"
        self.added, self.writes = [], []

    def add_sequence(self, sid):
        self.added.append(sid)

    def write_block(self, layer, sids, starts, k, v):
        self.writes.append((layer, tuple(sids), tuple(starts), k))
        if layer == 0:
            self.allocator.num_free -= -(-k // self.block_size)


class _Model:
    num_layers = 2

    def prompt_kv(self, n):
        return n, n


def _driver(cap=20, bs=4, gamma=3, max_batch=3):
    return SpecContinuousDriver(_KV(cap, bs), _Model(), gamma, max_batch)


def test_lifetime_blocks_bound_every_round():
    drv = _driver(bs=4, gamma=3)
    # prompt 10, budget 6: cache holds at most 10 + 6 - 2 = 14 tokens, +4 verify rows
    assert drv.lifetime_blocks(10, 6) == 5
    assert drv.lifetime_blocks(8, 1) == 3


def test_admission_in_arrival_order_with_reservation():
    drv = _driver(cap=20, bs=4, gamma=3, max_batch=3)
    res = DriverResult(3)
    due = [Request(0, 0, 10, 6), Request(1, 0, 40, 20), Request(2, 0, 4, 4)]
    waiting = drv._flush_arrivals(due, res)
    # request 0 holds 3 blocks and may claim 2 more: 20 - 5 = 15 left for the
    # queue; request 1 needs ceil(62 / 4) = 16, waits and holds back request 2
    assert [s.sid for s in drv.running] == [0]
    assert [r.sid for r in waiting] == [1, 2]
    assert drv.kv.added == [0]
    assert [(w[0], w[1], w[2]) for w in drv.kv.writes] == [(0, (0,), (0,)), (1, (0,), (0,))]
    s = drv.running[0]
    assert (s.length, s.generated, s.lifetime_blocks) == (10, 1, 5)
    assert res.admitted == 1


def test_batch_cap_and_unfittable_request():
    drv = _driver(cap=100, bs=4, gamma=3, max_batch=2)
    res = DriverResult(3)
    waiting = drv._flush_arrivals([Request(i, 0, 5, 5) for i in range(4)], res)
    assert [s.sid for s in drv.running] == [0, 1] and [r.sid for r in waiting] == [2, 3]
    with pytest.raises(ValueError):
        _driver(cap=8)._flush_arrivals([Request(9, 0, 40, 10)], DriverResult(3))


def test_mean_acceptance_follows_reference_definition():
    r = DriverResult(5, tokens_per_round=[1, 3, 6, 2])
    assert r.mean_tokens_per_round == 3.0
    assert r.mean_acceptance == 0.5


def test_poisson_requests_are_seeded_and_ordered():
    a = poisson_requests(50, 0.5, 512, 8192, 16, 64, seed=7)
    b = poisson_requests(50, 0.5, 512, 8192, 16, 64, seed=7)
    assert a == b
    assert [r.arrive_step for r in a] == sorted(r.arrive_step for r in a)
    assert all(512 <= r.prompt_len <= 8192 and 16 <= r.max_new_tokens <= 64 for r in a)
    assert len({r.sid for r in a}) == 50
