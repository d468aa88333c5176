"""GPU parity: decode-token append, seal and mean-key representative
(bit-exact bytes and fp32 bits against the oracle), page gather, the
synthetic generator and the copy-stream miss correction."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import device_kv, pool_numpy, status_tensor, to_dev
from paged_case import D, PAGE, make_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("local_tokens", [0, 32])
def test_append_seal_sequence_bit_exact(hip, local_tokens):
    """70 decode steps over 3 sequences with different starting tails."""
    case = make_case(200 + local_tokens, 3, 16, 8, [32 * 5 + 30, 32 * 2, 32 * 7 + 13], table_stride=16,
                     local_tokens=local_tokens)
    kv = device_kv(case)
    st = status_tensor()
    rng = np.random.default_rng(9)
    for step in range(70):
        k = (rng.standard_normal((3, 8, D)) * 2).astype(np.float32)
        v = (rng.standard_normal((3, 8, D)) * 2).astype(np.float32)
        if step == 3:
            k[0, 0, :4] = [65519.0, 65520.0, 1e-8, -3e-5]  # overflow / subnormal edges
        hip.append_seal(kv, to_dev(k), to_dev(v), local_tokens, status=st)
        O.paged_append(case.pool, PAGE, case.table, case.seq_len, k=k, v=v, batch=3, hkv=8, d=D)
        O.paged_seal(case.pool, PAGE, case.table, case.seq_len, case.sealed, case.generation, case.reps, 8,
                     case.rep_stride, 3, 16, 8, D, local_tokens)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    assert np.array_equal(kv.seq_len.cpu().numpy(), case.seq_len)
    assert np.array_equal(kv.sealed.cpu().numpy(), case.sealed)
    assert np.array_equal(kv.generation.cpu().numpy(), case.generation)
    assert np.array_equal(pool_numpy(kv), case.pool)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), case.reps.view(np.uint32))


def test_append_f16_raw_bits(hip):
    case = make_case(210, 2, 16, 8, [31, 64 + 5], table_stride=8)
    kv = device_kv(case)
    rng = np.random.default_rng(3)
    k16 = rng.integers(0, 65536, size=(2, 8, D)).astype(np.uint16)
    k16[(k16 & 0x7C00) == 0x7C00] = 0x3C00  # keep values finite
    v16 = rng.integers(0, 0x7BFF, size=(2, 8, D)).astype(np.uint16)
    hip.append_seal(kv, to_dev(k16.view(np.int16)).view(torch.uint16),
                    to_dev(v16.view(np.int16)).view(torch.uint16), 0)
    O.paged_append(case.pool, PAGE, case.table, case.seq_len, k16=k16, v16=v16, batch=2, hkv=8, d=D)
    O.paged_seal(case.pool, PAGE, case.table, case.seq_len, case.sealed, case.generation, case.reps, 8,
                 case.rep_stride, 2, 16, 8, D, 0)
    torch.cuda.synchronize()
    assert np.array_equal(pool_numpy(kv), case.pool)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), case.reps.view(np.uint32))


def test_seal_after_prefill_per_query_head_reps(hip):
    """Prefill wrote whole pages; one seal call seals every block and writes
    the same mean key to each query head of the group."""
    case = make_case(211, 2, 32, 8, [32 * 40 + 3, 32 * 9], rep_heads=32)
    kv = device_kv(case)
    kv.sealed.zero_()
    kv.generation.zero_()
    kv.reps.zero_()
    hip.seal(kv, 0)
    torch.cuda.synchronize()
    assert np.array_equal(kv.sealed.cpu().numpy(), case.sealed)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), case.reps.view(np.uint32))


@pytest.mark.parametrize("rep_heads,local_tokens,hq,hkv", [(8, 0, 16, 8), (8, 32, 16, 8), (16, 0, 16, 8),
                                                          (2, 0, 4, 2), (12, 32, 12, 6)])
def test_bulk_seal_from_partial_state(hip, rep_heads, local_tokens, hq, hkv):
    """The bulk seal (one workgroup per 16 blocks and KV head) from sealed
    counts part-way through the range, over chunk boundaries (0, 1, 15, 16,
    17, 33, 100 blocks to seal), at 8, 2 and 6 KV heads: representatives,
    sealed and generation bit-exact against the oracle's tail rule."""
    print(f"case: bulk seal rep_heads={rep_heads} local={local_tokens} hq={hq} hkv={hkv}", flush=True)
    lengths = [32 * 100 + 7, 32 * 17, 32 * 16 + 31, 31, 32 * 33, 32 * 61 + 1, 32 * 2]
    case = make_case(214 + local_tokens + rep_heads, len(lengths), hq, hkv, lengths, rep_heads=rep_heads,
                     local_tokens=local_tokens)
    start = np.array([0, 0, 1, 0, 3, 44, 1], np.int32)
    start = np.minimum(start, case.sealed)
    reps0 = np.random.default_rng(5).standard_normal(case.reps.shape).astype(np.float32)
    kv = device_kv(case)
    kv.sealed.copy_(to_dev(start))
    kv.generation.copy_(to_dev(start * 3))
    kv.reps.copy_(to_dev(reps0))
    st = status_tensor()
    hip.seal(kv, local_tokens, status=st)
    # oracle: the same start, the tail rule block by block
    sealed = start.copy()
    gen = start * 3
    reps = reps0.copy()
    O.paged_seal(case.pool, PAGE, case.table, case.seq_len, sealed, gen, reps, rep_heads, case.rep_stride,
                 case.batch, hq, hkv, D, local_tokens)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    assert np.array_equal(kv.sealed.cpu().numpy(), sealed)
    assert np.array_equal(kv.generation.cpu().numpy(), gen)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), reps.view(np.uint32))


@pytest.mark.parametrize("hole", ["page", "rep_stride"])
def test_bulk_seal_stops_at_capacity(hip, hole):
    """A block without a page (table entry -1) or past the representative
    capacity stops the bulk seal there, as the tail rule stops: the blocks
    before it are sealed bit-exact, nothing after it is written, the
    capacity bit is set and the counters stop at the hole."""
    lengths = np.array([32 * 60, 32 * 40], np.int32)
    if hole == "page":
        stop = 37
        case = make_case(215, 2, 16, 8, lengths)
        short = lengths.copy()
        short[0] = stop * PAGE
    else:
        # 62 pages per sequence, representative slots for 36 blocks only
        stop = 36
        short = np.array([32 * stop, 32 * stop], np.int32)
        case = make_case(215, 2, 16, 8, short, table_stride=62, rep_stride=stop)
    table = case.table.copy()
    if hole == "page":
        table[0, stop] = -1
    kv = device_kv(case)
    kv.block_table.copy_(to_dev(table))
    kv.seq_len.copy_(to_dev(lengths))
    kv.sealed.zero_()
    kv.generation.zero_()
    kv.reps.zero_()
    st = status_tensor()
    hip.seal(kv, 0, status=st)
    sealed = np.zeros(2, np.int32)
    gen = np.zeros(2, np.int32)
    reps = np.zeros_like(case.reps)
    O.paged_seal(case.pool, PAGE, case.table, short, sealed, gen, reps, 8, case.rep_stride, 2, 16, 8, D, 0)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_CAPACITY
    assert np.array_equal(kv.sealed.cpu().numpy(), sealed)
    assert np.array_equal(kv.generation.cpu().numpy(), gen)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), reps.view(np.uint32))


def test_capacity_is_flagged(hip):
    case = make_case(212, 1, 16, 8, [32 * 4 - 1], table_stride=4)
    kv = device_kv(case)
    st = status_tensor()
    z = torch.zeros((1, 8, D), dtype=torch.float32, device="cuda")
    hip.append_seal(kv, z, z, 0, status=st)   # fills the last page
    hip.append_seal(kv, z, z, 0, status=st)   # no page left: flagged, nothing written
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_CAPACITY
    assert int(kv.seq_len.item()) == 32 * 4


def test_gather_pages_bit_exact(hip):
    case = make_case(213, 2, 16, 8, [32 * 20, 32 * 10])
    kv = device_kv(case)
    pages = case.table[[0, 0, 1, 0], [3, 7, 2, 19]].astype(np.int32)
    out = torch.zeros((4, case.page_elems), dtype=torch.int16, device="cuda").view(torch.uint16)
    hip.gather_pages(kv.pool, kv.page_bytes, kv.num_pages, to_dev(pages), out)
    torch.cuda.synchronize()
    expect = np.zeros(4 * case.page_elems, np.uint16)
    O.lib().sao_pack_blocks(case.pool.ctypes.data, case.page_elems, pages.ctypes.data, 4, expect.ctypes.data)
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16).ravel(), expect)


@pytest.mark.parametrize("seed", [0, 77])
def test_synthetic_generator_matches_oracle(hip, seed):
    n = 1 << 20
    t16 = torch.empty(n, dtype=torch.int16, device="cuda").view(torch.uint16)
    t32 = torch.empty(4096, dtype=torch.float32, device="cuda")
    hip.fill_synthetic_f16(t16, seed, 12345)
    hip.fill_synthetic_f32(t32, seed, 999)
    torch.cuda.synchronize()
    assert np.array_equal(t16.view(torch.int16).cpu().numpy().view(np.uint16), O.synth_half(seed, 12345, n))
    assert np.array_equal(t32.cpu().numpy().view(np.uint32), O.synth_float(seed, 999, 4096).view(np.uint32))


def test_consume_checksum(hip):
    x = np.random.default_rng(1).standard_normal(2048).astype(np.float32)
    out = torch.zeros(1, dtype=torch.float32, device="cuda")
    hip.consume_checksum(to_dev(x), out)
    torch.cuda.synchronize()
    expect = np.float32(0)
    for i, xi in enumerate(x):
        expect = np.float32(expect + np.float32(xi * np.float32(np.float32(1.0) + np.float32(i % 17) * np.float32(0.001))))
    assert out.item() == float(expect)


def test_miss_correction_copy_stream(hip):
    """History prediction + correction (reference pipeline_main.cpp:686-717,
    305-331): missing blocks are copied from pinned host memory into the
    evicted slots on a copy stream; the compute stream waits on an event;
    the resident set equals the selection and the slot bytes equal the store."""
    rng = np.random.default_rng(4)
    n_blocks, slots = 64, 16
    page_elems = 32 * 2 * 8 * 128
    store = torch.from_numpy(rng.integers(0, 65536, size=(n_blocks, page_elems)).astype(np.uint16).view(np.int16))
    store = store.pin_memory()
    pool = torch.zeros((slots, page_elems), dtype=torch.int16, device="cuda")
    predicted = sorted(rng.choice(n_blocks, size=slots, replace=False).tolist())
    resident = list(predicted)  # slot i holds block resident[i]
    pool.copy_(store[predicted].cuda())
    copy_stream = torch.cuda.Stream()
    compute = torch.cuda.current_stream()
    done = torch.cuda.Event()
    done.record(copy_stream)  # materialise the event
    misses_total = 0
    for step in range(6):
        keep = rng.choice(resident, size=12, replace=False).tolist()
        fresh = rng.choice([b for b in range(n_blocks) if b not in resident], size=4, replace=False).tolist()
        oracle_set = sorted(keep + fresh)
        hits, misses, repl = hip.compare_prediction(resident, oracle_set)
        st, ohits, omisses, orepl = O.compare_prediction(resident, oracle_set)
        assert (hits, misses, repl) == (ohits, omisses, orepl)
        hip.fill_pages_async(pool, page_elems * 2, repl, store.data_ptr(), misses, copy_stream, done)
        hip.stream_wait_event(compute, done)
        for slot, blk in zip(repl, misses):
            resident[slot] = blk
        misses_total += len(misses)
        assert sorted(resident) == oracle_set
        compute.synchronize()
        assert torch.equal(pool.cpu(), store[resident])
    assert misses_total == 24


def test_miss_fill_gather_kernel_from_pinned_memory(hip):
    """The one-launch fill reads pinned host pages through their device
    mapping; slot bytes equal the store; bad pages are flagged, not read."""
    rng = np.random.default_rng(8)
    n_blocks, slots = 48, 20
    page_elems = 32 * 2 * 8 * 128
    store = torch.from_numpy(rng.integers(0, 65536, size=(n_blocks, page_elems)).astype(np.uint16).view(np.int16))
    store = store.pin_memory()
    pool = torch.zeros((slots, page_elems), dtype=torch.int16, device="cuda")
    dst = np.array([3, 7, 0, 19, 11], np.int32)
    src = np.array([40, 2, 17, 33, 5], np.int64)
    copy_stream = torch.cuda.Stream()
    done = torch.cuda.Event()
    done.record(copy_stream)
    st = status_tensor()
    hip.fill_pages_gather_async(pool, page_elems * 2, slots, to_dev(dst), store.data_ptr(), n_blocks, to_dev(src),
                                len(dst), copy_stream, done, status=st)
    hip.stream_wait_event(torch.cuda.current_stream(), done)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    got = pool.cpu()
    for d_, s_ in zip(dst, src):
        assert torch.equal(got[d_], store[s_])
    untouched = sorted(set(range(slots)) - set(dst.tolist()))
    assert (got[untouched] == 0).all()
    bad = np.array([slots + 5], np.int32)
    hip.fill_pages_gather_async(pool, page_elems * 2, slots, to_dev(bad), store.data_ptr(), n_blocks, to_dev(src[:1]),
                                1, copy_stream, done, status=st)
    copy_stream.synchronize()
    assert int(st.item()) & hip.STATUS_BAD_PAGE
    st.zero_()
    far = np.array([n_blocks + 3], np.int64)  # beyond the store: skipped, never read
    hip.fill_pages_gather_async(pool, page_elems * 2, slots, to_dev(dst[:1]), store.data_ptr(), n_blocks, to_dev(far),
                                1, copy_stream, done, status=st)
    copy_stream.synchronize()
    assert int(st.item()) & hip.STATUS_BAD_PAGE


@pytest.mark.parametrize("pinned", [True, False])
def test_pages_to_host_staging(hip, pinned):
    """Seal writeback staging: pool pages to pinned host memory (one kernel
    writing through the device mapping) or to pageable memory (one copy per
    page), ordered after an event of the compute stream; bytes equal."""
    import numpy as np
    import torch
    rng = np.random.default_rng(71)
    npages = 300  # two launches of the pinned path (256 ids each at most)
    kv = hip.PagedKV(1, 16, 8, 4, num_pages=npages)
    bits = rng.integers(0, 65536, size=tuple(kv.pool.shape), dtype=np.uint16).view(np.int16)
    kv.pool.view(torch.int16).copy_(torch.from_numpy(bits).cuda())
    pages = rng.permutation(npages)[:260].astype(np.int32)
    pb = kv.page_bytes
    dst = torch.zeros(len(pages) * pb, dtype=torch.uint8)
    if pinned:
        dst = dst.pin_memory()
    copy = torch.cuda.Stream()
    after, done = torch.cuda.Event(), torch.cuda.Event()
    after.record(torch.cuda.current_stream())
    done.record(copy)
    print(f"case: pinned={pinned} pages={len(pages)}", flush=True)
    hip.pages_to_host_async(kv.pool, pb, npages, pages, dst, copy, after_event=after, done_event=done)
    done.synchronize()
    got = dst.numpy().reshape(len(pages), pb)
    ref = kv.pool.view(torch.uint8).view(npages, pb).cpu().numpy()[pages]
    assert np.array_equal(got, ref)
    with pytest.raises(hip.SaHipError, match="outside"):
        hip.pages_to_host_async(kv.pool, pb, npages, [npages], dst, copy)
