"""Hot-channel policy simulations (host bookkeeping, no GPU): counterpart of the reference's
tests/test_hot_cache.py. Expected values are hand-computed from each policy's rule."""
import pytest

from soinfer.offload import hot_cache as HC


def test_static_policy_ties_keep_lower_index_and_clamp():
    assert HC.StaticFrequencyPolicy([5, 5, 5, 1], cache_size=2).hot_set == frozenset({0, 1})
    p = HC.StaticFrequencyPolicy([3, 1], cache_size=10)
    assert p.cache_size == 2 and p.hot_set == frozenset({0, 1})
    r = HC.StaticFrequencyPolicy([5, 5, 5, 1], cache_size=2).simulate([[0], [1], [2], [3], [0, 1, 2]])
    assert (r.hits, r.total) == (4, 7) and r.hit_rate == pytest.approx(4 / 7)


@pytest.mark.parametrize("trace,size,hits", [
    ([[0], [1], [2], [1], [0]], 2, 1),           # 0,1 fill; 2 evicts 0; 1 hits; 0 misses (evicts 2)
    ([[0], [0], [0]], 0, 0),                      # no cache, no hits
    ([[0], [1], [2]] * 3, 3, 6),                  # every channel fits: one miss each, then hits
    ([[0, 1, 2], [1, 3]], 2, 1),                  # a token selecting more than the cache: 1 still hits next token
    ([[0, 1], [1, 0], [2], [0]], 2, 2),           # token 1 hits both (0, then 1 most recent); 2 evicts 0; 0 misses
])
def test_lru_hand_computed(trace, size, hits):
    r = HC.LRUPolicy(size).simulate(trace)
    assert r.hits == hits and r.total == sum(len(t) for t in trace)


def test_lru_batch_lookup_before_insert():
    # token 1 = [1, 2]: with cache {0, 1} (0 least recent), 1 hits first, then 2 evicts 0, so token 2's 1 hits
    r = HC.LRUPolicy(2).simulate([[0, 1], [1, 2], [1]])
    assert r.hits == 2


def test_lfu_hand_computed():
    # 0, 1 fill; 0 hits (freq 2); 2 evicts the lower-frequency 1
    r = HC.LFUDecayPolicy(2, decay_every=1000).simulate([[0], [1], [0], [2]])
    assert (r.hits, r.total) == (1, 4)
    # tie at frequency 1: 2 evicts the higher index (1), so 0 still hits and 1 misses
    r = HC.LFUDecayPolicy(2, decay_every=1000).simulate([[0], [1], [2], [0], [1]])
    assert (r.hits, r.total) == (1, 5)
    with pytest.raises(ValueError):
        HC.LFUDecayPolicy(2, decay=0.0)


def test_lfu_decay_lets_an_old_favourite_go():
    """Channel 0 is selected 10 times, then never. Without decay it survives the later eviction contests
    (the final [0] hits); with decay 0.3 per token its count fades below channel 2's and it is evicted when 1
    arrives, so the final [0] misses. Both runs hit 11 times before that token."""
    trace = [[0]] * 10 + [[2]] + [[1]] * 3 + [[3]] + [[0]]
    keep = HC.LFUDecayPolicy(2, decay=1.0, decay_every=1).simulate(trace)
    fade = HC.LFUDecayPolicy(2, decay=0.3, decay_every=1).simulate(trace)
    assert (keep.hits, fade.hits) == (12, 11)
    assert keep.total == fade.total == len(trace)


def test_compare_policies_runs_all_three_per_size():
    trace = [[0, 1], [1, 2], [0, 1], [3], [1]]
    res = HC.compare_policies(trace, [1, 2], decay_every=2)
    assert [r.policy for r in res] == ["static", "lru", "lfu_decay"] * 2
    assert [r.cache_size for r in res] == [1, 1, 1, 2, 2, 2]
    assert all(r.total == 8 for r in res)
    # static with the trace's own counts (0:2, 1:4, 2:1, 3:1): size 1 keeps {1} -> 4 hits; size 2 {0, 1} -> 6
    assert (res[0].hits, res[3].hits) == (4, 6)


def test_lru_heap_equals_a_list_replay_on_random_traces():
    """The heap-based LRU against a plain recency list replayed by hand (look up the whole token, then insert its
    misses ascending, evicting from the front), over random traces with tokens larger than the cache."""
    import random

    rng = random.Random(5)
    for size in (0, 1, 3, 8, 20):
        trace = [rng.sample(range(40), rng.randint(1, 25)) for _ in range(60)]
        recency, hits = [], 0
        for tok in trace:
            tok = sorted(tok)
            for c in tok:
                if c in recency:
                    hits += 1
                    recency.remove(c)
                    recency.append(c)
            for c in tok:
                if c not in recency and size > 0:
                    if len(recency) >= size:
                        recency.pop(0)
                    recency.append(c)
        r = HC.LRUPolicy(size).simulate(trace)
        assert r.hits == hits and r.total == sum(len(t) for t in trace), size
