"""Device memory planner (memory_planner_t; the reference's
src/memory_planner.cpp:33-337), planned on the optimized graph without a GPU:
lifetimes over the executed plan, in-place outputs, concat aliasing and
best-fit slots. The invariant checked is the one a plan must satisfy to be
correct: two pooled tensors live at the same node position occupy disjoint
bytes, unless one is written over the other on purpose (in place) or lives
inside it (a concatenation's part)."""
import numpy as np
import pytest

from nnr_amd import graph as G
from nnr_amd import synth


def family(entries, i):
    """The entry whose slot i's bytes belong to (in-place / concat parents)."""
    while entries[i]["kind"] != "slot":
        i = entries[i]["parent"]
    return i


def check_plan(stats, entries):
    assert stats["intermediates"] == len(entries)
    assert stats["pool_bytes"] <= stats["unpooled_bytes"]
    fam = [family(entries, i) for i in range(len(entries))]
    for i, e in enumerate(entries):
        assert e["first"] <= e["last"]
        assert e["offset"] + e["bytes"] <= stats["pool_bytes"], e
        if e["kind"] == "slot":
            assert e["offset"] % 256 == 0
        elif e["kind"] == "inplace":
            p = entries[e["parent"]]
            assert p["offset"] == e["offset"] and p["bytes"] == e["bytes"]
            assert p["last"] >= e["first"]
        else:
            p = entries[e["parent"]]
            assert p["offset"] <= e["offset"] and e["offset"] + e["bytes"] <= p["offset"] + p["bytes"]
            assert p["first"] <= e["first"] and e["last"] <= p["last"]
    # live at the same position => disjoint bytes, unless of one family (and
    # then only an in-place chain or a part inside its concatenation)
    n = len(entries)
    first = np.array([e["first"] for e in entries])
    last = np.array([e["last"] for e in entries])
    lo = np.array([e["offset"] for e in entries], dtype=np.int64)
    hi = lo + np.array([e["bytes"] for e in entries], dtype=np.int64)
    for i in range(n):
        live = (first <= last[i]) & (last >= first[i])
        mem = (lo < hi[i]) & (hi > lo[i])
        for j in np.nonzero(live & mem)[0]:
            if j == i:
                continue
            assert fam[i] == fam[j], (entries[i], entries[j])
            if entries[i]["kind"] == "concat" and entries[j]["kind"] == "concat":
                assert entries[i]["parent"] != entries[j]["parent"], (entries[i], entries[j])


def plan_of(g, **kw):
    s = G.Session(g, device=False, memory_planning=True, **kw)
    return s.memory_plan()


@pytest.mark.parametrize("name,build", [
    ("resnet50", lambda: synth.resnet50(batch=2, hw=64, seed=14)),
    ("mobilenetv2", lambda: synth.mobilenetv2(batch=2, hw=64, seed=17)),
    ("bert", lambda: synth.bert(batch=2, seq=32, layers=2)),
    ("qoperator", lambda: synth.qoperator_net(batch=2, hw=21)),
])
def test_plan_invariants(name, build):
    stats, entries = plan_of(build())
    check_plan(stats, entries)
    assert stats["slots"] < stats["intermediates"]
    # sharing pays: the arena is a fraction of one allocation per tensor
    assert stats["pool_bytes"] < 0.6 * stats["unpooled_bytes"], stats


def test_resnet50_adds_in_place():
    """Without the conv epilogue fusion (not applied by a plan of the
    optimized graph), each residual QLinearAdd reads both operands for the
    last time and writes over one of them."""
    stats, entries = plan_of(synth.resnet50(batch=2, hw=64, seed=14))
    assert stats["inplace"] == 16
    check_plan(stats, entries)


def test_concat_parts_alias_the_output():
    stats, entries = plan_of(synth.concat_net(batch=1))
    check_plan(stats, entries)
    assert stats["concat"] == 2 and stats["inplace"] == 1
    by = {e["name"]: e for e in entries}
    cat = [e for e in entries if e["kind"] == "concat"]
    parent = entries[cat[0]["parent"]]
    assert sorted(e["offset"] - parent["offset"] for e in cat) == [0, 16 * 8 * 8]
    # the QLinearAdd of the concatenation with itself writes over it
    assert [e for e in entries if e["kind"] == "inplace"][0]["parent"] == entries.index(parent)
    assert len(by) == len(entries)


def test_concat_not_aliased_past_batch_one():
    """With a batch dimension before the axis the parts are strided inside
    the output: no aliasing (memory_planner.cpp:165-170)."""
    stats, entries = plan_of(synth.concat_net(batch=2))
    check_plan(stats, entries)
    assert stats["concat"] == 0


def test_checker_catches_overlap():
    """The invariant check itself: two live tensors placed on the same bytes
    fail it."""
    stats, entries = plan_of(synth.resnet50(batch=2, hw=64, seed=14))
    bad = [dict(e) for e in entries]
    a = next(i for i, e in enumerate(bad) if e["kind"] == "slot")
    b = next(i for i, e in enumerate(bad) if i != a and e["kind"] == "slot"
             and e["first"] <= bad[a]["last"] and e["last"] >= bad[a]["first"])
    bad[b]["offset"] = bad[a]["offset"]
    with pytest.raises(AssertionError):
        check_plan(stats, bad)
