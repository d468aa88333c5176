"""The oracle against committed reference outputs (tests/golden/): the
reference's own attention_reference, select_shared_blocks,
build_local_causal_representatives and float_to_half
(cpp/src/attention_reference.cpp:11-96, cpp/src/selection.cpp:12-147), run
by tests/golden/make_golden.py through oracle/_ref.  Bit-exact, and
independent of the reference checkout (these run wherever the fixtures are)."""
import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)

from cases import (ATTENTION, CODEC, REPRESENTATIVES, SELECTION, attention_inputs, codec_inputs,  # noqa: E402
                   representative_inputs, selection_inputs, sha)

GOLD = np.load(os.path.join(HERE, "reference_outputs.npz"), allow_pickle=False)
META = json.load(open(os.path.join(HERE, "reference_outputs.json")))["cases"]


def test_every_case_has_a_golden():
    names = ([f"attention/{n}" for n in ATTENTION] + [f"selection/{n}" for n in SELECTION] +
             [f"representatives/{n}" for n in REPRESENTATIVES] + [f"codec/{n}" for n in CODEC])
    assert sorted(names) == sorted(META)


@pytest.mark.parametrize("name", sorted(ATTENTION))
def test_attention_matches_reference_bits(oracle_lib, name):
    c = ATTENTION[name]
    kv, q = attention_inputs(c)
    assert sha(kv, q) == META[f"attention/{name}"]["input_sha256"], "input generator drifted"
    scale = float(np.float32(1.0) / np.sqrt(np.float32(c["d"])))
    got = oracle_lib.attention_reference(kv, q, c["tokens"], c["hq"], c["hkv"], c["d"], scale)
    assert np.array_equal(got.view(np.uint32), GOLD[f"attention/{name}"])


@pytest.mark.parametrize("name", sorted(SELECTION))
def test_selection_matches_reference(oracle_lib, name):
    c = SELECTION[name]
    q, reps = selection_inputs(c)
    assert sha(q, reps) == META[f"selection/{name}"]["input_sha256"], "input generator drifted"
    ids, scores = oracle_lib.select_shared_blocks(q, reps, c["heads"], c["blocks"], 128, c["budget"], c["init"],
                                                  c["local"])
    assert ids.tolist() == GOLD[f"selection/{name}/ids"].tolist()
    assert np.array_equal(scores.view(np.uint32), GOLD[f"selection/{name}/scores"])


@pytest.mark.parametrize("name", sorted(REPRESENTATIVES))
def test_representatives_match_reference(oracle_lib, name):
    c = REPRESENTATIVES[name]
    pq, kv = representative_inputs(c)
    assert sha(pq, kv) == META[f"representatives/{name}"]["input_sha256"], "input generator drifted"
    vals, offs = oracle_lib.local_causal_representatives(pq, kv, c["tokens"], c["hq"], c["hkv"], 128, 32,
                                                         c["window"], c["topk"])
    assert np.array_equal(offs.astype(np.int64), GOLD[f"representatives/{name}/offsets"])
    assert np.array_equal(vals.view(np.uint32), GOLD[f"representatives/{name}/values"])


def test_fixture_selection_golden_is_not_trivial():
    """The tie and zero cases pick lowest ids among equals, as a stable sort does."""
    assert GOLD["selection/zeros/ids"].tolist() == [0, 1, 2, 3, 4, 5, 6, 7, 48, 49]


@pytest.mark.parametrize("name", sorted(CODEC))
def test_float_to_half_matches_reference(oracle_lib, name):
    x = codec_inputs(CODEC[name])
    assert sha(x) == META[f"codec/{name}"]["input_sha256"], "input generator drifted"
    L = oracle_lib.lib()
    got = np.array([L.sao_float_to_half(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, GOLD[f"codec/{name}"])
