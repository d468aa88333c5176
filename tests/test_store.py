"""The main KV store (include/sa_store.h) on the CPU: the reference's block
offsets, round trips through the worker threads, O_DIRECT where the file
system has it, argument and I/O errors, and the commit marker."""
import os

import numpy as np
import pytest

import solidattention_amd as sa


def deterministic_block(global_block, nbytes):
    """Bytes of block `global_block` in the reference's deterministic store
    (cpp/src/uring_reader.cpp:130-140): (block * 17 + index * 13) & 0xff."""
    idx = np.arange(nbytes, dtype=np.int64)
    return ((global_block * 17 + idx * 13) & 0xFF).astype(np.uint8)


def aligned(nbytes):
    """A 4096-byte aligned numpy buffer (O_DIRECT)."""
    raw = np.zeros(nbytes + 4096, np.uint8)
    off = (-raw.ctypes.data) % 4096
    return raw[off: off + nbytes]


@pytest.mark.parametrize("direct", [True, False])
def test_round_trip_and_offsets(tmp_path, direct):
    layers, bpl, bb = 3, 10, 8192
    path = str(tmp_path / "main-kv-store.bin")
    st = sa.MainStore(path, layers, bpl, bb, create=True, direct=direct, threads=4)
    assert st.nbytes == layers * bpl * bb == os.path.getsize(path)
    src = aligned(5 * bb)
    for i in range(5):
        src[i * bb:(i + 1) * bb] = deterministic_block(100 + i, bb)
    st.write(1, [7, 0, 9, 3, 4], src)
    st.sync()
    # the file holds block b of layer l at (l * blocks_per_layer + b) * block_bytes
    raw = np.fromfile(path, np.uint8)
    for i, blk in enumerate([7, 0, 9, 3, 4]):
        off = (1 * bpl + blk) * bb
        assert np.array_equal(raw[off: off + bb], deterministic_block(100 + i, bb)), blk
    dst = aligned(3 * bb)
    st.read(1, [4, 7, 3], dst)
    for i, src_i in enumerate([4, 0, 3]):
        assert np.array_equal(dst[i * bb:(i + 1) * bb], deterministic_block(100 + src_i, bb))
    st.close()


def test_async_batches_many_threads(tmp_path):
    """Several batches in flight at once, waited in another order."""
    layers, bpl, bb = 2, 64, 4096
    path = str(tmp_path / "s.bin")
    st = sa.MainStore(path, layers, bpl, bb, create=True, threads=8)
    src = aligned(layers * bpl * bb)
    for layer in range(layers):
        for b in range(bpl):
            g = layer * bpl + b
            src[g * bb:(g + 1) * bb] = deterministic_block(g, bb)
    w = [st.submit_writes(layer, range(bpl), src[layer * bpl * bb:(layer + 1) * bpl * bb]) for layer in range(layers)]
    for bid in reversed(w):
        st.wait(bid)
    rng = np.random.default_rng(0)
    order = [rng.permutation(bpl)[:20] for _ in range(layers)]
    dsts = [aligned(20 * bb) for _ in range(layers)]
    r = [st.submit_reads(layer, order[layer], dsts[layer]) for layer in range(layers)]
    for bid in r:
        st.wait(bid)
    for layer in range(layers):
        for i, b in enumerate(order[layer]):
            assert np.array_equal(dsts[layer][i * bb:(i + 1) * bb], deterministic_block(layer * bpl + int(b), bb))
    st.close()


def test_lifecycle_store_closed_form(tmp_path):
    """The reference's P1.3b.0 main store: 28 layers, capacity 16 + 512/32 + 1
    blocks of 32 x 2 x 8 x 128 FP16 = 131072 bytes: 121,110,528 bytes
    (artifacts/runs/P1.3b.0-native-main-store-lifecycle-metrics.json)."""
    st = sa.MainStore(str(tmp_path / "m.bin"), 28, 16 + (512 + 31) // 32 + 1, 32 * 2 * 8 * 128 * 2, create=True)
    assert st.nbytes == 121110528
    st.close()


def test_argument_and_io_errors(tmp_path):
    path = str(tmp_path / "e.bin")
    st = sa.MainStore(path, 2, 4, 4096, create=True, direct=True)
    buf = aligned(2 * 4096)
    with pytest.raises(sa.SaHipError, match="layer"):
        st.write(2, [0], buf)
    with pytest.raises(sa.SaHipError, match="block"):
        st.read(0, [4], buf)
    with pytest.raises(sa.SaHipError, match="block"):
        st.read(0, [-1], buf)
    # an unaligned buffer goes through the bounce buffer under O_DIRECT
    src = aligned(4096)
    src[:] = deterministic_block(3, 4096)
    st.write(1, [2], src)
    odd = np.zeros(4097, np.uint8)
    st.read(1, [2], odd[1:])
    assert np.array_equal(odd[1:], src)
    assert st.bounced == (1 if st.direct else 0)
    st.close()
    # an existing file shorter than its declared layout: a short read is an error
    with open(tmp_path / "short.bin", "wb") as f:
        f.write(b"\0" * 4096)
    st2 = sa.MainStore(str(tmp_path / "short.bin"), 1, 4, 4096, create=False, direct=False)
    with pytest.raises(sa.SaHipError, match="short"):
        st2.read(0, [2], buf)
    st2.close()
    with pytest.raises(sa.SaHipError):
        sa.MainStore(str(tmp_path / "missing" / "x.bin"), 1, 1, 4096, create=True)
    with pytest.raises(sa.SaHipError, match="4096"):
        sa.MainStore(str(tmp_path / "y.bin"), 1, 1, 1000, create=True, direct=True)


def test_commit_marker_replaces_atomically(tmp_path):
    """online_seal_main.cpp:59-70: body to name.tmp, fsync, rename, fsync of
    the directory; the old marker is replaced whole and no .tmp remains."""
    sa.commit_marker(str(tmp_path), "generation.json", '{"generation":1,"block_id":16,"layers":28}\n')
    assert (tmp_path / "generation.json").read_text() == '{"generation":1,"block_id":16,"layers":28}\n'
    sa.commit_marker(str(tmp_path), "generation.json", '{"generation":2}\n')
    assert (tmp_path / "generation.json").read_text() == '{"generation":2}\n'
    assert not (tmp_path / "generation.json.tmp").exists()
    with pytest.raises(sa.SaHipError):
        sa.commit_marker(str(tmp_path), "a/b", "x")
    with pytest.raises(sa.SaHipError):
        sa.commit_marker(str(tmp_path / "nope"), "g.json", "x")
