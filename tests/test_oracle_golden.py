"""The oracle against the reference's published golden values.

Goldens (reference artifacts/runs/*-metrics.json and docs/):
  C2.1  selected ids [0,8,13,15], representative offset hash
        7873450381430813043, selected-vs-dense cosine 0.987693
        (docs/cpp-versions/C2.1-infllm-selection-uring.md:40-42,66-67)
  P1.1  dense_oracle_block_recall 0.809152, dense_selected_attention_mass
        0.264404, 742 misses / hit rate 0.585938 over 16 steps x 28 layers
        (artifacts/runs/P1.1-infllm-history-correction-metrics.json)
  P1.0  346 misses / hit rate 0.80692 with the closed-form oracle sets
        (artifacts/runs/P1.0-history-correction-metrics.json)
  P1.3b.0  448 sealed blocks, 7168 representative audits, tail 32,
        generation 16, store 121110528 B
        (artifacts/runs/P1.3b.0-native-main-store-lifecycle-metrics.json)
"""
import numpy as np
import pytest


def fnv_offsets(offsets):
    h = 1469598103934665603
    for o in np.asarray(offsets).ravel():
        h ^= int(o)
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


@pytest.fixture(scope="module")
def c2(oracle_lib):
    O = oracle_lib
    kv, pq = O.fixture_c2(512, 16, 8, 128)
    reps, offsets = O.local_causal_representatives(pq, kv, 512, 16, 8, 128, 32, 32, 4)
    query = pq.reshape(16, 512, 128)[:, 511, :].copy()
    return kv, pq, reps, offsets, query


def test_c21_representative_offset_hash(c2):
    _, _, _, offsets, _ = c2
    assert fnv_offsets(offsets) == 7873450381430813043


def test_c21_selected_ids(c2, oracle_lib):
    _, _, reps, _, query = c2
    ids, _ = oracle_lib.select_shared_blocks(query, reps, 16, 16, 128, 4, 1, 1)
    assert ids.tolist() == [0, 8, 13, 15]


def test_c21_selected_vs_dense_cosine(c2, oracle_lib):
    kv, _, reps, _, query = c2
    O = oracle_lib
    ids, _ = O.select_shared_blocks(query, reps, 16, 16, 128, 4, 1, 1)
    block = 32 * 2 * 8 * 128
    packed = np.concatenate([kv[i * block:(i + 1) * block] for i in ids])
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    sparse = O.attention_reference(packed, query, 128, 16, 8, 128, scale).ravel().astype(np.float64)
    dense = O.attention_reference(kv, query, 512, 16, 8, 128, scale).ravel().astype(np.float64)
    cos = sparse @ dense / np.sqrt((sparse @ sparse) * (dense @ dense))
    assert f"{cos:.6f}" == "0.987693"


def test_p11_dense_audit(c2, oracle_lib):
    kv, pq, reps, _, _ = c2
    mass, recall = oracle_lib.p1_dense_audit(kv, pq, reps, 16, 28)
    assert f"{mass:.6f}" == "0.264404"
    assert f"{recall:.6f}" == "0.809152"


def _history_run(blocks_fn, steps=16, layers=28, oracle_lib=None):
    """pipeline_main.cpp:760-850: prediction = last step's set for the layer."""
    history = [blocks_fn(0, layer) for layer in range(layers)]
    predicted_total = hits_total = misses_total = 0
    for step in range(steps):
        for layer in range(layers):
            predicted = history[layer]
            oracle_set = blocks_fn(step, layer)
            st, hits, misses, slots = oracle_lib.compare_prediction(predicted, oracle_set)
            assert st == 0
            assert len(misses) == len(slots)
            predicted_total += len(predicted)
            hits_total += hits
            misses_total += len(misses)
            history[layer] = oracle_set
    return predicted_total, hits_total, misses_total


def test_p10_history_correction_counts(oracle_lib):
    pred, hits, misses = _history_run(oracle_lib.oracle_blocks, oracle_lib=oracle_lib)
    assert (pred, hits, misses) == (1792, 1446, 346)
    assert f"{hits / pred:.5f}" == "0.80692"


def test_p11_history_correction_counts(c2, oracle_lib):
    _, pq, reps, _, _ = c2
    O = oracle_lib
    pq3 = pq.reshape(16, 512, 128)

    def blocks(step, layer):
        pos = 512 - 1 - ((step * 17 + layer * 11) % 256)
        ids, _ = O.select_shared_blocks(pq3[:, pos, :].copy(), reps, 16, 16, 128, 4, 1, 1)
        return ids.tolist()

    pred, hits, misses = _history_run(blocks, oracle_lib=O)
    assert (pred, misses) == (1792, 742)
    assert f"{hits / pred:.6f}" == "0.585938"


def test_p13b0_lifecycle(oracle_lib):
    st, r = oracle_lib.run_synthetic_lifecycle(28, 512)
    assert st == 0, "sealed block bytes differ from the readback closed form"
    assert r.sealed_blocks == 448
    assert r.representative_head_audits == 7168
    assert r.resident_tail_tokens == 32
    assert r.generation == 16
    assert r.store_bytes == 121110528


def test_stale_ticket_self_test(oracle_lib):
    """pipeline_main.cpp:1065-1072: a ticket of generation 11 is stale at 12."""
    import ctypes as C
    blocks = (C.c_size_t * 4)(0, 1, 2, 15)
    L = oracle_lib.lib()
    assert not L.sao_valid_ticket(3, 7, 11, blocks, 3, 7, 12, blocks)
    assert L.sao_valid_ticket(3, 7, 12, blocks, 3, 7, 12, blocks)


def test_compare_prediction_cardinality_mismatch(oracle_lib):
    # a prediction with a duplicate cannot be corrected slot-for-slot
    st, _, _, _ = oracle_lib.compare_prediction([0, 0, 2, 15], [0, 1, 2, 15])
    assert st != 0


def test_topk_argmax_python_test_indices(oracle_lib):
    """The reference's tail test (tests/test_kv_lifecycle.py:22-37) expects
    representative indices [7, 9, 11, 13] for scores 10/9/8/7 at those tokens."""
    import numpy as np
    scores = np.zeros(32, np.float32)
    scores[[7, 9, 11, 13]] = [10, 9, 8, 7]
    top = np.zeros(4, np.uint64)
    oracle_lib.lib().sao_topk_argmax(scores.ctypes.data, 32, 4, top.ctypes.data)
    assert top.tolist() == [7, 9, 11, 13]
    # ties resolve to the first maximum, as the argmax-first loop does
    flat = np.ones(32, np.float32)
    oracle_lib.lib().sao_topk_argmax(flat.ctypes.data, 32, 4, top.ctypes.data)
    assert top.tolist() == [0, 1, 2, 3]
