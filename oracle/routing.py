"""ORACLE - test infrastructure only. Compares two runs' mixture-of-experts routing decisions.

A router (reference chroma/models/gpt_oss.py:243-263) ranks bfloat16 gate logits with ``torch.topk``
(sorted, ties to the lower expert id: chroma/_src/codegen/gpu.py:300-337). The device and the oracle
compute those logits with different (equally exact) orders of their float sums, so the same logit can
round to neighbouring bfloat16 values in the two runs, and two experts whose logits lie within a few
bfloat16 spacings of each other may swap ranks. Expert ids are held bit-exact everywhere else.

``compare_routing`` takes both runs' gate logits and expert ids over a sequence of positions and:

* counts the decisions (position, layer) whose ordered expert ids agree;
* sets apart *tie reorders*: the same experts, where every rank that differs holds two experts whose
  logits are exactly equal in both runs. Their softmax weights are then equal too, so the reorder only
  permutes the order of the combine's sum. The reference CPU backend orders exact ties as
  ``std::nth_element`` leaves them (chroma/_src/codegen/cpu/kernels.h:172-179; its own test calls tie
  order unspecified, tests/test_runtime.py:175-189), the reference GPU rule takes the lower id; each
  reorder records whether the first run (the device) took the lower id;
* for every other decision that differs (a *flip*), pairs the two runs' experts rank by rank and
  measures, in each run's own logits, the gap between the two experts of every differing pair in
  bfloat16 spacings at the row's scale (the spacing of the row's largest |logit|: a logit's final
  rounding and the float sums before it carry absolute errors of about that size whatever the logit's
  own magnitude, so a gap between two logits near zero is not measured in their own tiny spacing). The
  flip is *explained* only when every pair is within ``bound_ulps`` in both runs' own logits: a flip
  both runs see as a near-tie;
* checks that the first run's ids are exactly the top-k of its own logits (descending, ties to the lower
  id, the reference GPU rule) at every decision, and the second run's up to the order of exact ties;
* measures the two runs' gate logits against each other over the decisions not downstream of a flip,
  as the largest difference in the same row-scale spacings;
* leaves out of the count the decisions downstream of a flip: position p at a later layer than a flip at
  position p0 <= p (causal attention carries p0's changed state into every later position), reported
  apart with their own agreement.

``downstream_of(flips, position, layers)`` says whether a position's final hidden state (and its logits)
depends on a flip: a flip at that position, or at an earlier position in any layer but the last.
"""

from __future__ import annotations

from typing import Dict, List, Sequence

import numpy as np


def bf16_spacing(values: np.ndarray) -> np.ndarray:
    """Distance from |x| to the next larger bfloat16 (8 significant bits): 2^(floor(log2|x|) - 7), with
    the subnormal spacing 2^-133 as the floor."""
    magnitude = np.maximum(np.abs(np.asarray(values, dtype=np.float64)), 2.0**-126)
    return np.exp2(np.floor(np.log2(magnitude)) - 7)


def row_spacing(logits: np.ndarray) -> float:
    """The bfloat16 spacing at a row's scale: that of its largest magnitude."""
    return float(bf16_spacing(np.max(np.abs(logits))))


def gap_ulps(logits: np.ndarray, a: int, b: int) -> float:
    """|logits[a] - logits[b]| in bfloat16 spacings at the row's scale (``row_spacing``)."""
    return abs(float(logits[a]) - float(logits[b])) / row_spacing(logits)


def top_ids(logits: np.ndarray, k: int) -> np.ndarray:
    """Ordered top-k ids of each row: values descending, ties to the lower id (NaN not expected here)."""
    return np.argsort(-np.asarray(logits, dtype=np.float64), axis=-1, kind="stable")[..., :k]


def compare_routing(hip_ids: np.ndarray, hip_logits: np.ndarray, ref_ids: np.ndarray, ref_logits: np.ndarray,
                    *, bound_ulps: float = 2.0) -> Dict:
    """Both runs' decisions: ids [layers, positions, k] (int64) and logits [layers, positions, experts]
    (float32, widened from bfloat16). Returns the agreement summary described in the module docstring."""
    hip_ids, ref_ids = np.asarray(hip_ids), np.asarray(ref_ids)
    hip_logits, ref_logits = np.asarray(hip_logits, dtype=np.float32), np.asarray(ref_logits, dtype=np.float32)
    if hip_ids.shape != ref_ids.shape or hip_logits.shape != ref_logits.shape or hip_ids.shape[:2] != hip_logits.shape[:2]:
        raise ValueError(f"routing shapes differ: {hip_ids.shape} {ref_ids.shape} {hip_logits.shape} {ref_logits.shape}")
    layers, positions, k = hip_ids.shape
    own = top_ids(hip_logits, k)
    hip_selection = [(int(p), int(l)) for l, p in zip(*np.nonzero((own != hip_ids).any(-1)))]
    # the second run up to the order of exact ties: its chosen values are the top-k values in descending
    # order, and its ids are distinct
    ref_top = np.take_along_axis(ref_logits, top_ids(ref_logits, k), -1)
    ref_chosen = np.take_along_axis(ref_logits, ref_ids, -1)
    distinct = np.array([[len(set(row.tolist())) == k for row in layer] for layer in ref_ids], dtype=bool).reshape(layers, positions)
    bad = (ref_top != ref_chosen).any(-1) | ~distinct
    ref_selection = [(int(p), int(l)) for l, p in zip(*np.nonzero(bad))]
    worst_logit = 0.0
    flips: List[Dict] = []
    ties: List[Dict] = []
    compared = matched = downstream = downstream_matched = 0
    # earliest position with a (first-class) flip at any layer before the current one
    first_flip = positions
    for layer in range(layers):
        layer_flips = []
        for position in range(positions):
            same = bool(np.array_equal(hip_ids[layer, position], ref_ids[layer, position]))
            if position >= first_flip:
                downstream += 1
                downstream_matched += same
                continue
            compared += 1
            matched += same
            worst_logit = max(worst_logit, float(np.max(np.abs(hip_logits[layer, position] - ref_logits[layer, position])))
                              / row_spacing(ref_logits[layer, position]))
            if same:
                continue
            pairs = []
            for rank, (h, r) in enumerate(zip(hip_ids[layer, position], ref_ids[layer, position])):
                if h == r:
                    continue
                pairs.append({"rank": rank, "hip_expert": int(h), "ref_expert": int(r),
                              "hip_gap_ulps": round(gap_ulps(hip_logits[layer, position], int(h), int(r)), 2),
                              "ref_gap_ulps": round(gap_ulps(ref_logits[layer, position], int(h), int(r)), 2)})
            if set(hip_ids[layer, position].tolist()) == set(ref_ids[layer, position].tolist()) and all(
                    hip_logits[layer, position, p["hip_expert"]] == hip_logits[layer, position, p["ref_expert"]]
                    and ref_logits[layer, position, p["hip_expert"]] == ref_logits[layer, position, p["ref_expert"]] for p in pairs):
                # among exactly tied experts, the first run's order is ascending id (the lower-id rule)
                tied = [int(e) for e in hip_ids[layer, position] if any(e in (p["hip_expert"], p["ref_expert"]) for p in pairs)]
                ties.append({"position": position, "layer": layer, "hip_ids": [int(i) for i in hip_ids[layer, position]],
                             "ref_ids": [int(i) for i in ref_ids[layer, position]], "hip_lower_id_first": tied == sorted(tied)})
                continue
            explained = all(p["hip_gap_ulps"] <= bound_ulps and p["ref_gap_ulps"] <= bound_ulps for p in pairs)
            layer_flips.append({"position": position, "layer": layer, "hip_ids": [int(i) for i in hip_ids[layer, position]],
                                "ref_ids": [int(i) for i in ref_ids[layer, position]], "pairs": pairs, "explained": explained})
        flips.extend(layer_flips)
        if layer_flips:
            first_flip = min(first_flip, min(f["position"] for f in layer_flips))
    return {
        "decisions": layers * positions,
        "compared": compared,
        "matched": matched,
        "tie_reorders": ties,
        "agreement": round((matched + len(ties)) / compared, 6) if compared else None,
        "flips": flips,
        "unexplained": sum(not f["explained"] for f in flips),
        "bound_ulps": bound_ulps,
        "downstream": downstream,
        "downstream_matched": downstream_matched,
        "hip_selection_mismatches": hip_selection,
        "ref_selection_mismatches": ref_selection,
        "logit_max_diff_ulps": round(worst_logit, 3),
    }


def downstream_of(flips: Sequence[Dict], position: int, layers: int) -> bool:
    """Whether the final hidden state of ``position`` depends on one of ``flips``: a flip at that
    position (any layer), or at an earlier position in a layer before the last (whose changed state
    reaches ``position`` through a later layer's attention)."""
    return any(f["position"] == position or (f["position"] < position and f["layer"] < layers - 1) for f in flips)
