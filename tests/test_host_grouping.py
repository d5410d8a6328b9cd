"""CPU tests of libtfq's host grouping (tfq_group_pairs_host), the product's
restatement of PrefillMoEGrouping.groupTokenExpertPairs
(S/Kernels/Prefill/MoE/PrefillMoEGrouping.swift:91-192): the reference's
known-answer tests (T/Kernels/Prefill/PrefillMoEGroupingTests.swift) and
agreement with the oracle on random and skewed inputs. No GPU involved."""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import synth
from edgeexpert_amd.ops import GroupingError, PAIR_DTYPE, PrefillMoEGrouping, PrefillRouter

G = PrefillMoEGrouping.group_token_expert_pairs


def _pairs(rows):
    a = np.zeros(len(rows), PAIR_DTYPE)
    for i, r in enumerate(rows):
        a[i] = r
    return a


def _tuples(arr):
    return [tuple(int(v) for v in x) for x in arr]


def test_known_answer_sort_offsets_counts_groups_tiles():
    # PrefillMoEGroupingTests.swift:5-53
    rows = [(0, 3, 0, 10), (0, 1, 1, 11), (0, 4, 2, 12), (1, 1, 0, 13), (1, 3, 1, 14), (1, 2, 2, 15),
            (2, 4, 0, 16), (2, 3, 1, 17), (2, 1, 2, 18), (3, 5, 0, 19), (3, 1, 1, 20), (3, 4, 2, 21)]
    g = G(_pairs(rows[::-1]), 4, 3, 6, 2)
    assert list(g["sorted"]["expert"]) == [1, 1, 1, 1, 2, 3, 3, 3, 4, 4, 4, 5]
    assert [[int(p["token"]), int(p["rank"])] for p in g["sorted"]] == [
        [0, 1], [1, 0], [2, 2], [3, 1], [1, 2], [0, 0], [1, 1], [2, 1], [0, 2], [2, 0], [3, 2], [3, 0]]
    assert list(g["offsets"]) == [0xFFFFFFFF, 0, 4, 5, 8, 11]
    assert list(g["counts"]) == [0, 4, 1, 3, 3, 1]
    assert _tuples(g["groups"]) == [(1, 0, 4), (2, 4, 1), (3, 5, 3), (4, 8, 3), (5, 11, 1)]
    assert _tuples(g["tiles"]) == [(0, 2, 0, 5), (2, 2, 5, 6), (4, 1, 11, 1)]


def test_deterministic_across_input_order_and_weight_bits_preserved():
    # PrefillMoEGroupingTests.swift:55-82
    tm = [(0, 2, 0, 101), (0, 1, 1, 102), (1, 2, 0, 103), (1, 0, 1, 104), (2, 1, 0, 105), (2, 2, 1, 106)]
    sh = [tm[5], tm[1], tm[3], tm[0], tm[4], tm[2]]
    a, b = G(_pairs(tm), 3, 2, 3, 2), G(_pairs(sh), 3, 2, 3, 2)
    for k in ("sorted", "offsets", "counts", "groups", "tiles"):
        assert np.array_equal(a[k], b[k])
    assert list(a["sorted"]["weight_bits"]) == [104, 102, 105, 101, 103, 106]


def test_sort_keys_order_tiles():
    # PrefillMoEGroupingTests.swift:84-115
    rows = [(0, 1, 0, 10), (0, 2, 1, 20), (1, 3, 0, 30), (1, 1, 1, 11), (2, 2, 0, 21), (2, 3, 1, 31)]
    g = G(_pairs(rows), 3, 2, 4, 2, expert_sort_keys=[0, 30, 10, 20])
    assert list(g["groups"]["expert"]) == [2, 3, 1]
    assert list(g["sorted"]["expert"]) == [2, 2, 3, 3, 1, 1]
    assert list(g["offsets"]) == [0xFFFFFFFF, 4, 0, 2]
    assert _tuples(g["tiles"]) == [(0, 2, 0, 4), (2, 1, 4, 2)]


@pytest.mark.parametrize("rows,args,kw,name,values", [
    ([(0, 0, 0, 1)], (1, 1, 1, 17), {}, "invalidTileExpertCount", (17, 0)),
    ([(0, 2, 0, 1)], (1, 1, 2, 1), {}, "expertOutOfRange", (2, 0)),
    ([(0, 0, 0, 1), (0, 1, 0, 2)], (1, 2, 2, 1), {}, "duplicateTokenRank", (0, 0)),
    ([(0, 0, 0, 1)], (1, 1, 2, 1), {"expert_sort_keys": [0]}, "expertSortKeyCountMismatch", (2, 1)),
    ([(0, 0, 0, 1)], (2, 1, 2, 1), {}, "pairCountMismatch", (2, 1)),
    ([(1, 0, 0, 1)], (1, 1, 2, 1), {}, "tokenOutOfRange", (1, 0)),
    ([(0, 0, 1, 1)], (1, 1, 2, 1), {}, "rankOutOfRange", (1, 0)),
    ([], (-1, 1, 2, 1), {}, "invalidQueryCount", (-1, 0)),
    ([], (0, 0, 2, 1), {}, "invalidTopK", (0, 0)),
    ([], (0, 1, 0, 1), {}, "invalidNumExperts", (0, 0)),
])
def test_rejects_invalid_metadata(rows, args, kw, name, values):
    # PrefillMoEGroupingTests.swift:117-173 plus every other error case
    with pytest.raises(GroupingError) as ei:
        G(_pairs(rows), *args, **kw)
    assert ei.value.name == name and ei.value.values == values
    with pytest.raises(oracle.GroupingError) as eo:
        oracle.group_pairs(_pairs(rows).astype(oracle.PAIR_DTYPE), *args,
                           sort_keys=kw.get("expert_sort_keys"))
    assert eo.value.name == name and eo.value.values == values


def test_t32_pressure():
    # PrefillMoEGroupingTests.swift:175-203
    rows = [(t, (t + r * 7) % 74, r, t * 8 + r) for t in range(32) for r in range(8)]
    g = G(_pairs(rows), 32, 8, 128, 16)
    assert g["sorted"].size == 256 and g["groups"].size <= 74
    assert all(t["group_count"] <= 16 and t["pair_count"] > 0 for t in g["tiles"])


@pytest.mark.parametrize("T,k,E,tile,keys", [(512, 8, 128, 16, False), (37, 4, 16, 3, True),
                                             (1, 8, 256, 1, False)])
def test_matches_oracle_on_skewed_routing(T, k, E, tile, keys):
    idx, w = synth.zipf_routing(3, f"grp/{T}", T, E, k)
    pairs = PrefillRouter.make_token_expert_pairs(idx, w, T, k)
    rng = np.random.RandomState(T)
    pairs = pairs[rng.permutation(pairs.size)]
    sk = rng.randint(0, 10, E).astype(np.uint64) if keys else None
    a = G(pairs, T, k, E, tile, expert_sort_keys=sk)
    b = oracle.group_pairs(pairs.astype(oracle.PAIR_DTYPE), T, k, E, tile, sort_keys=sk)
    assert a["sorted"].tobytes() == b["sorted"].tobytes()
    for key in ("offsets", "counts"):
        assert np.array_equal(a[key], b[key])
    assert a["groups"].tobytes() == b["groups"].tobytes()
    assert a["tiles"].tobytes() == b["tiles"].tobytes()
