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


@pytest.mark.gpu
@pytest.mark.parametrize("per_channel", [False, True])
def test_fused_chain_values_get_no_memory(dev, per_channel):
    """A fused chain's stage-to-stage values (a QLinearMatMul's uint8 result
    before its DequantizeLinear; MatMulInteger's int32 result, the Cast and
    scale-Mul outputs before the bias) exist only inside the kernel: they
    get no arena slot, while what a stage reads from outside the chain (the
    activation scale the per-channel epilogue reads on the device) stays
    live at the fused node. (The chains are formed by operators built on
    the device.)"""
    g = synth.bert(batch=2, seq=32, layers=2, per_channel=per_channel)
    s = G.Session(g, memory_planning=True)
    plan = s.plan()
    stats, entries = s.memory_plan()
    check_plan(stats, entries)
    by = {e["name"]: e for e in entries}
    inner, reads, chains = set(), [], 0
    for i, p in enumerate(plan):
        if not p["fused_chain"]:
            continue
        chains += 1
        nodes = [g.node_by_name(c) for c in p["fused_chain"]]
        outs = set(p["outputs"])
        if nodes[0].inputs[0] not in outs:
            inner.add(nodes[0].inputs[0])
        inner |= {t for nd in nodes for t in nd.outputs if t not in outs}
        reads += [(i, t) for nd in nodes for t in nd.inputs
                  if t not in inner and t not in g.initializers]
    assert chains >= 8
    assert not inner & set(by), sorted(inner & set(by))
    for i, t in reads:
        if t in by:
            assert by[t]["first"] <= i <= by[t]["last"], (t, i, by[t])
