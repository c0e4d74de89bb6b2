"""Routing probes and the routing-agreement checker, on the CPU.

* ``oracle.routing.compare_routing`` against hand-built decisions: agreement, flips explained only by a
  near-tie in both runs' own logits, a planted wrong choice reported unexplained, and the decisions
  downstream of a flip left out of the count.
* ``export_cached(..., routing=True)`` probes: outputs 0-2 bit-identical to the plain export's on the
  oracle, the extra outputs equal to the model's own router decisions (eager torch), and the ``Decoder``
  collecting them per run only when asked to (reference chroma/models/gpt_oss.py:243-263).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from chroma_amd import Decoder
from chroma_amd.models.cached import CachedTransformer, export_cached
from oracle import compile_cpu
from oracle.routing import bf16_spacing, compare_routing, downstream_of, gap_ulps
from tests.test_decoder import small_model


def test_bf16_spacing_known_answers():
    np.testing.assert_array_equal(bf16_spacing(np.array([1.0, 1.5, 1.9921875, 2.0, 0.75, -3.0])),
                                  [2.0**-7, 2.0**-7, 2.0**-7, 2.0**-6, 2.0**-8, 2.0**-6])
    assert gap_ulps(np.array([1.0, 1.0 + 2**-7, 1.0 + 2**-5]), 0, 1) == 1.0
    assert gap_ulps(np.array([1.0, 1.0 + 2**-7, 1.0 + 2**-5]), 2, 0) == 4.0
    assert gap_ulps(np.array([-2.0, 2.0]), 0, 1) == 4.0 / 2**-6
    # gaps are measured in the spacing at the row's scale, not at the two logits' own magnitude
    assert gap_ulps(np.array([0.1, 0.1 + 2**-11, 2.5]), 0, 1) == 2.0**-11 / 2.0**-6


def decisions(logits: np.ndarray, k: int) -> np.ndarray:
    """Ordered top-k ids per row, ties to the lower id (the reference's rule)."""
    return np.argsort(-logits, axis=-1, kind="stable")[..., :k]


def test_compare_routing_counts_and_explains_flips():
    rng = np.random.default_rng(0)
    layers, positions, experts, k = 3, 6, 8, 2
    # well separated logits: multiples of 1/8 at magnitude ~1 are 16 bf16 spacings apart
    logits = np.stack([[rng.permutation(experts) / 8.0 + 1.0 for _ in range(positions)] for _ in range(layers)]).astype(np.float32)
    ids = decisions(logits, k)
    same = compare_routing(ids, logits, ids.copy(), logits.copy())
    assert same["agreement"] == 1.0 and same["compared"] == layers * positions and not same["flips"]

    # a near-tie: at (position 4, layer 1) the 2nd and 3rd experts sit one spacing apart, in opposite
    # order in the two runs; the 2nd-ranked expert differs, and both runs see the pair as a near-tie
    hip, ref = logits.copy(), logits.copy()
    second, third = np.argsort(-logits[1, 4], kind="stable")[1:3]
    top = logits[1, 4, second]
    hip[1, 4, second], hip[1, 4, third] = top, top - 2**-7
    ref[1, 4, second], ref[1, 4, third] = top - 2**-7, top
    result = compare_routing(decisions(hip, k), hip, decisions(ref, k), ref)
    assert [(f["position"], f["layer"], f["explained"]) for f in result["flips"]] == [(4, 1, True)]
    assert result["flips"][0]["pairs"][0]["hip_gap_ulps"] == result["flips"][0]["pairs"][0]["ref_gap_ulps"] == 1.0
    # downstream of (4, 1): positions 4 and 5 of layer 2 are left out of the count
    assert result["downstream"] == 2 and result["compared"] == layers * positions - 2
    assert result["matched"] == result["compared"] - 1 and result["unexplained"] == 0

    # a planted mistake: the device picks an expert its own logits rank far below (16 spacings)
    wrong = decisions(logits, k)
    wrong[0, 2, 1] = np.argsort(-logits[0, 2], kind="stable")[2]
    result = compare_routing(wrong, logits, ids, logits)
    assert result["unexplained"] == 1 and result["flips"][0]["pairs"][0]["hip_gap_ulps"] >= 8
    assert result["downstream"] == 2 * 4  # positions 2..5 of layers 1 and 2

    # an exact tie ordered differently: the same experts, equal logits in both runs; not a flip, nothing
    # downstream is left out, and the device's lower-id-first order is recorded
    tied = logits.copy()
    first, second = np.argsort(-logits[2, 1], kind="stable")[:2]
    tied[2, 1, second] = tied[2, 1, first]
    low, high = sorted((int(first), int(second)))
    hip_ids, ref_ids = decisions(tied, k), decisions(tied, k)
    ref_ids[2, 1] = [high, low]
    result = compare_routing(hip_ids, tied, ref_ids, tied)
    assert not result["flips"] and result["downstream"] == 0 and result["matched"] == result["compared"] - 1
    assert result["agreement"] == 1.0
    assert [(t["position"], t["layer"], t["hip_lower_id_first"]) for t in result["tie_reorders"]] == [(1, 2, True)]
    assert not compare_routing(ref_ids, tied, hip_ids, tied)["tie_reorders"][0]["hip_lower_id_first"]
    # the same swap where one run's logits differ by a spacing is a flip (explained: 1 spacing)
    near = tied.copy()
    near[2, 1, high] -= 2**-7 * (1 if abs(near[2, 1, high]) < 2 else 2)
    result = compare_routing(hip_ids, near, ref_ids, tied)
    assert len(result["flips"]) == 1 and result["flips"][0]["explained"] and not result["tie_reorders"]

    # each run's ids are checked against its own logits: the first run's exactly (lower id on ties), the
    # second's up to the order of exact ties
    assert not result["hip_selection_mismatches"] and not result["ref_selection_mismatches"]
    assert compare_routing(ref_ids, tied, hip_ids, tied)["hip_selection_mismatches"] == [(1, 2)]
    assert not compare_routing(ref_ids, tied, hip_ids, tied)["ref_selection_mismatches"]
    broken = ids.copy()
    broken[1, 3] = broken[1, 3][::-1]  # a device that returns its top two in the wrong order
    assert compare_routing(broken, logits, ids, logits)["hip_selection_mismatches"] == [(3, 1)]
    assert compare_routing(ids, logits, broken, logits)["ref_selection_mismatches"] == [(3, 1)]
    assert compare_routing(ids, logits, ids, logits + 2**-6)["logit_max_diff_ulps"] == 2.0

    # shapes must agree
    with pytest.raises(ValueError):
        compare_routing(ids[:, :3], logits, ids, logits)


def test_downstream_of():
    flips = [{"position": 3, "layer": 0}, {"position": 5, "layer": 2}]
    layers = 3
    assert not downstream_of(flips, 2, layers)
    assert downstream_of(flips, 3, layers)  # its own flip
    assert downstream_of(flips, 4, layers)  # position 3's flip in layer 0 reaches it through layers 1-2
    assert downstream_of([{"position": 5, "layer": 2}], 5, layers)
    assert not downstream_of([{"position": 5, "layer": 2}], 6, layers)  # a last-layer flip of another position


@pytest.fixture(scope="module")
def probe_pair(tmp_path_factory):
    model = small_model(8)
    context = 7
    root = tmp_path_factory.mktemp("probe")
    graphs = {(steps, routing): export_cached(model, context, steps, routing=routing) for steps in (context, 1) for routing in (False, True)}
    programs = {key: compile_cpu(graph, root / f"{key[0]}_{int(key[1])}") for key, graph in graphs.items()}
    return model, context, programs


def test_routing_probe_keeps_the_arithmetic_and_reports_the_model_routing(probe_pair):
    model, context, programs = probe_pair
    steps = context
    generator = torch.Generator().manual_seed(1)
    layers, kv_heads, head_dim = len(model.block), model.block[0].attn.num_key_value_heads, model.block[0].attn.head_dim
    cache = (layers, context, kv_heads, head_dim)
    times = torch.arange(steps) + 3
    keys_times = torch.arange(context)
    allowed = keys_times[None, :] < 3  # three cached positions, then the causal band over the new keys
    mask = torch.full((steps, context + steps), -float("inf"))
    mask[:, :context][allowed.expand(steps, -1)] = 0
    mask[:, context:] = torch.triu(torch.full((steps, steps), -float("inf")), diagonal=1)
    inputs = (torch.randint(0, 31, (steps,), generator=generator), times.float(), torch.randn(cache, generator=generator) * 0.3,
              torch.randn(cache, generator=generator) * 0.3, mask, mask.clone(), torch.tensor([steps - 1]))
    arrays = [x.numpy() for x in inputs]
    plain = programs[(steps, False)](*arrays)
    probe = programs[(steps, True)](*arrays)
    assert len(plain) == 3 and len(probe) == 5
    for a, b in zip(plain, probe[:3]):
        np.testing.assert_array_equal(a, b)
    with torch.no_grad():
        eager = CachedTransformer(model, routing=True)(*inputs)
    gate_logits, expert_ids = probe[3], probe[4]
    assert gate_logits.shape == (layers, steps, model.block[0].mlp.num_experts) and expert_ids.shape == (layers, steps, 2)
    np.testing.assert_array_equal(expert_ids, eager[4].numpy())
    np.testing.assert_allclose(gate_logits, eager[3].numpy(), rtol=2e-5, atol=2e-6)


def test_decoder_collects_extra_outputs_only_when_asked(probe_pair):
    """A probe pair needs ``extra_outputs=True``; its logits equal the plain pair's bit for bit, and the
    decisions gathered from ``extras`` over every run equal the routing of an eager causal forward whose
    windows are clipped to the cache (the reference decoder test's construction, test_decoder.py:82-113)."""
    import copy

    model, context, programs = probe_pair
    with pytest.raises(ValueError, match="seven inputs and three outputs"):
        Decoder(programs[(context, True)], programs[(1, True)])
    with pytest.raises(ValueError, match="pair"):
        Decoder(programs[(context, True)], programs[(1, False)], extra_outputs=True)
    tokens = (np.arange(7) * 5 + 2) % 31
    reference = copy.deepcopy(model)
    for block in reference.block:
        block.attn.sliding_window = min(block.attn.sliding_window or context, context)
    gates = []
    hooks = [block.mlp.gate.register_forward_hook(lambda m, i, o: gates.append(o.detach())) for block in reference.block]
    with torch.no_grad():
        reference(torch.from_numpy(tokens))
    for hook in hooks:
        hook.remove()
    want = np.stack([torch.topk(g, 2, dim=-1).indices.numpy() for g in gates])  # [layers, positions, 2]
    got = []
    with Decoder(programs[(context, True)], programs[(1, True)], sliding_window=3, extra_outputs=True) as probe, \
            Decoder(programs[(context, False)], programs[(1, False)], sliding_window=3) as plain:
        for start, end in ((0, 5), (5, 6), (6, 7)):
            np.testing.assert_array_equal(probe.append(tokens[start:end]), plain.append(tokens[start:end]))
            runs = probe.extras
            assert [(first, count) for first, count, _ in runs] == [(start, end - start)]
            for _, count, (gate_logits, expert_ids) in runs:
                assert gate_logits.shape == (len(model.block), context if count > 1 else 1, 4)
                got.append(expert_ids[:, :count])
        assert plain.extras == []
    np.testing.assert_array_equal(np.concatenate(got, axis=1), want)
