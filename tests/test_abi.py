"""CPU checks of the C ABI (include/qattn.h / libqattn.so) that need no GPU: the library loads
and exports every declared symbol, the host planner's work list and figures, argument
validation, and the kernel's key-tile iteration (compiled for the host from the same
attn_common.h) against the oracle's mask, bit for bit.
"""
import ctypes
import subprocess

import numpy as np
import pytest

FAKE = 0x100000  # aligned, non-NULL stand-in device addresses for host-only planning


def _desc(qattn, lengths, mask=1, P=176, W=432, **kw):
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return qattn.make_desc(FAKE, FAKE, FAKE, FAKE, cu, mask, P, W, **kw)


def test_library_exports_every_declared_symbol(qattn):
    declared = qattn.header_symbols()
    assert len(declared) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", qattn.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    lib = qattn.lib()
    for s in declared:
        assert getattr(lib, s) is not None


def test_abi_version(qattn):
    assert qattn.lib().qattn_abi_version() == 9


def test_create_without_gpu_fails_cleanly(qattn):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(qattn.QattnError) as e:
        qattn.Context(0)
    assert e.value.code in (qattn.ENODEV, qattn.EHIP)
    assert qattn.lib().qattn_last_error(None)


@pytest.mark.parametrize("lengths,mask", [([50], 1), ([500] * 16, 1), ([5000], 1), ([1500], 1),
                                          ([10, 150, 64, 65, 1], 0), ([5000] * 4, 1), ([500] * 16, 0),
                                          ([3000, 700, 9000], 1), ([2048] * 3, 0)])
def test_planner_covers_every_tile_once_in_balanced_slots(qattn, oracle, lengths, mask):
    d = _desc(qattn, lengths, mask)
    entries, info = qattn.plan_describe(d)
    slots = qattn.plan_slots(d)
    want = {(int(np.sum(lengths[:s])), L, qb, (s << 4) | g)
            for s, L in enumerate(lengths) for qb in range((L + 63) // 64) for g in range(8)}
    got = [tuple(int(x) for x in e) for e in entries]
    assert {e[:4] for e in got} == want and len(want) == info.work_items
    # every item's key tiles are covered exactly once: by one whole entry, or by the chunks of
    # one split (split >= 0) whose part fields agree (chunk ci of n, partial index first + ci)
    by_item = {}
    for e in got:
        by_item.setdefault(e[:4], []).append(e)
    splits, partials = set(), set()
    for item, es in by_item.items():
        n = len(_tiles(item[2], item[1], mask))
        cover = sorted((e[4], e[5]) for e in es)
        assert cover[0][0] == 0 and cover[-1][1] == n
        assert all(x[1] == y[0] and x[0] < x[1] for x, y in zip(cover, cover[1:]))
        assert cover[-1][0] < cover[-1][1]
        if len(es) == 1:
            assert es[0][6] == -1 and es[0][7] == 0
            continue
        assert len({e[6] for e in es}) == 1 and es[0][6] >= 0 and es[0][6] not in splits
        splits.add(es[0][6])
        parts = sorted((e[7] & 15, (e[7] >> 4) & 15, e[7] >> 8) for e in es)
        assert len(es) <= 8  # the merge kernel combines up to 8 chunks in one pass
        assert [p[0] for p in parts] == list(range(len(es)))
        assert all(p[1] == len(es) for p in parts) and len({p[2] for p in parts}) == 1
        first = parts[0][2]
        assert not partials & set(range(first, first + len(es)))
        partials |= set(range(first, first + len(es)))
    assert info.split_items == len(splits)
    assert partials == set(range(len(partials)))
    # slot structure: offsets cover the list; slot b holds only KV heads g with g % 8 == b % 8
    # (workgroup b runs on XCD b % 8); at most 512 slots (256 CUs x 2)
    assert slots[0] == 0 and slots[-1] == len(got) and np.all(np.diff(slots) >= 0)
    assert info.slots == len(slots) - 1 <= 512
    cost = lambda e: 4 * (e[5] - e[4]) + 13  # the planner's cost model (quarter tiles)
    loads = np.array([sum(cost(e) for e in got[slots[b]:slots[b + 1]]) for b in range(len(slots) - 1)])
    for b in range(len(slots) - 1):
        assert all((e[3] & 15) % 8 == b % 8 for e in got[slots[b]:slots[b + 1]])
    # balance: no slot exceeds its XCD group's mean load by more than one maximal entry
    for g in range(8):
        grp = [e for e in got if (e[3] & 15) % 8 == g]
        if not grp:
            continue
        used = loads[g::8][loads[g::8] > 0]
        assert used.max() <= sum(cost(e) for e in grp) / len(used) + max(cost(e) for e in grp)
    # figures
    pairs = sum(oracle.mask_pairs(L, mask) for L in lengths)
    assert info.tokens == sum(lengths)
    assert info.pairs == pairs
    assert info.flops == 8192 * pairs
    assert info.bytes == 12288 * sum(lengths)
    assert info.tile_pairs >= pairs


def test_planner_splits_only_when_it_pays(qattn):
    # 16 x 500 full causal balances exactly without splitting (q-blocks pair up to 9 tiles)
    _, info = qattn.plan_describe(_desc(qattn, [500] * 16, 0))
    assert info.split_items == 0
    # 1 x 5000 sparse: 79 items per KV head on 64 slots -> some items are split
    entries, info = qattn.plan_describe(_desc(qattn, [5000], 1))
    assert info.split_items > 0
    slots = qattn.plan_slots(_desc(qattn, [5000], 1))
    loads = [sum(e[5] - e[4] for e in entries[slots[b]:slots[b + 1]]) for b in range(len(slots) - 1)]
    assert max(loads) <= 16  # tiles per slot, against 22 for whole items


@pytest.mark.parametrize("lengths,mask", [([500] * 16, 0), ([5000], 1), ([5000] * 4, 1)])
def test_planner_gives_second_workgroups_less_work(qattn, lengths, mask):
    # Slots 256..511 are the second workgroup on their CU and run slower while the first is
    # resident: the planner balances finish times (load x 1.3 for them), not loads.
    d = _desc(qattn, lengths, mask)
    entries, _ = qattn.plan_describe(d)
    slots = qattn.plan_slots(d)
    n = len(slots) - 1
    assert n == 512

    def cost(b):
        es = entries[slots[b]:slots[b + 1]]
        return 18 + sum(4 * (e[5] - e[4]) + 13 for e in es)

    first = [cost(b) for b in range(256)]
    second = [cost(b) for b in range(256, 512)]
    assert np.mean(second) < np.mean(first)
    span = max(max(first) * 1000, max(second) * 1300)
    even = max(max(first), max(second)) * 1300  # what equal loads would give at best
    assert span <= even


def test_planner_slot_count_follows_the_limit(qattn):
    d = _desc(qattn, [500] * 16, 1)
    assert len(qattn.plan_slots(d, 64)) - 1 == 64
    assert len(qattn.plan_slots(d, 8)) - 1 == 8
    small = _desc(qattn, [50], 1)  # 8 items: one per KV head, one slot each
    assert len(qattn.plan_slots(small)) - 1 == 8


def _tiles(qb, L, mask, P=176, W=432):
    q0, q1 = qb * 64, min(L, qb * 64 + 64) - 1
    last = q1 // 64
    if mask == 0:
        return list(range(last + 1))
    ps, ws = min(L, P), min(L, W)
    keep = set(range(min(last + 1, (ps + 63) // 64)))
    keep |= set(range(max(0, q0 - ws + 1) // 64, last + 1))
    return sorted(keep)


def test_planner_sparse_tile_count_closed_form(qattn):
    # 1 x 5000, prefix 176 / window 432, 64-key tiles: block qb (rows 64qb..64qb+63) visits the
    # 3 prefix tiles plus tiles floor((64qb-431)/64) .. qb.
    entries, info = qattn.plan_describe(_desc(qattn, [5000]))
    assert info.work_items == 79 * 8
    assert info.pairs == 2855472
    # every block past the prefix region visits at most 3 + 8 + 1 tiles
    assert max(len(_tiles(qb, 5000, 1)) for qb in range(79)) <= 12


def test_planner_o_last_bytes(qattn):
    _, info = qattn.plan_describe(_desc(qattn, [5000] * 4, o_last=FAKE))
    assert info.bytes == 12288 * 20000 + 4096 * 4


@pytest.mark.parametrize("bad,needle", [
    (dict(lengths=[5, 3], cu=[0, 5, 4]), "non-decreasing"),
    (dict(lengths=[5], cu=[1, 6]), "cu_seqlens[0]"),
    (dict(lengths=[5], q_row_stride=2052), "multiples of 8"),
    (dict(lengths=[5], k_row_stride=512), "too small"),
    (dict(lengths=[5], v_offset=3), "multiples of 8"),
    (dict(lengths=[5], mask=7), "unknown mask"),
    (dict(lengths=[5], P=0, W=0), "both 0"),
    (dict(lengths=[5], P=-1), ">= 0"),
    (dict(lengths=[5], misalign=True), "aligned"),
])
def test_validation_rejects_before_launch(qattn, bad, needle):
    lengths = bad.pop("lengths")
    cu = bad.pop("cu", None)
    misalign = bad.pop("misalign", False)
    d = _desc(qattn, lengths, mask=bad.pop("mask", 1), P=bad.pop("P", 176), W=bad.pop("W", 432), **bad)
    if cu is not None:
        d._cu = np.asarray(cu, np.int32)
        d.cu_seqlens = d._cu.ctypes.data
        d.nseq = len(cu) - 1
    if misalign:
        d.k = FAKE + 2
    with pytest.raises(qattn.QattnError) as e:
        qattn.plan_describe(d)
    assert e.value.code == qattn.EINVAL
    assert needle in str(e.value)


def test_validation_nseq_zero_and_null(qattn):
    d = _desc(qattn, [5])
    d.nseq = 0
    with pytest.raises(qattn.QattnError):
        qattn.plan_describe(d)
    d = _desc(qattn, [5])
    d.q = None
    with pytest.raises(qattn.QattnError):
        qattn.plan_describe(d)


def test_validation_rejects_sequences_beyond_32bit_offsets(qattn):
    d = _desc(qattn, [300000], v_row_stride=4096)
    with pytest.raises(qattn.QattnError) as e:
        qattn.plan_describe(d)
    assert "2 GiB" in str(e.value)
    qattn.plan_describe(_desc(qattn, [200000]))  # 200000 x 2048 x 2 B < 2 GiB


def test_empty_sequences_are_skipped(qattn):
    items, info = qattn.plan_describe(_desc(qattn, [0, 7, 0, 0, 70]))
    assert info.tokens == 77 and info.work_items == 8 * (1 + 2)
    assert {int(i[0]) for i in items} == {0, 7}


@pytest.mark.parametrize("L", [1, 2, 16, 31, 32, 33, 63, 64, 65, 127, 175, 176, 177, 431, 432, 433,
                               500, 607, 608, 609, 700, 1500, 5000])
def test_kernel_key_iteration_matches_reference_mask(qattn, oracle, L):
    got = qattn.plan_mask(L)
    want = oracle.mask_bits(L)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("L,mask,P,W", [(300, 0, 0, 0), (129, 1, 7, 50), (200, 1, 0, 33), (200, 1, 64, 1),
                                         (333, 1, 1, 200), (1000, 1, 300, 64)])
def test_kernel_key_iteration_other_masks(qattn, oracle, L, mask, P, W):
    assert np.array_equal(qattn.plan_mask(L, mask, P, W), oracle.mask_bits(L, mask, P, W))


def test_kernel_mask_cases_sweep(qattn, oracle):
    # Every tile-mask case (tile_mask_case / tile_case_keeps, the compares the kernel executes)
    # over a grid of lengths, prefixes and windows around the tile and wavefront boundaries.
    n = 0
    for P in (0, 1, 5, 31, 32, 33, 63, 64, 65, 100, 176):
        for W in (0, 1, 2, 31, 32, 33, 63, 64, 65, 97, 432):
            if P == 0 and W == 0:
                continue
            for L in (1, 33, 64, 65, 129, 191, 257, 300):
                assert np.array_equal(qattn.plan_mask(L, 1, P, W), oracle.mask_bits(L, 1, P, W)), (L, P, W)
                n += 1
    assert n == 960


def test_q4_compact_bytes(qattn, oracle):
    f = qattn.lib().qattn_q4_compact_bytes
    assert f(1024, 4096) == 128 * 32 * 32 * 20
    assert f(96, 70) == 3 * 3 * 32 * 20
    assert f(32, 1) == 32 * 20
    assert f(33, 1) == -1 and f(0, 5) == -1 and f(64, 0) == -1
    # the oracle's packer writes exactly that many bytes
    packed, k, n = oracle.pack_q40_tile32([(96, 70, bytes(70 * 3 * 18))])
    assert packed.size == f(96, 70)


def test_consumer_and_projection_entry_points_reject_null_before_any_device_use(qattn):
    # No context, no device: both entry points validate on the host and return EINVAL.
    import numpy as np
    lib = qattn.lib()
    cu = np.array([0, 3], np.int32)
    assert lib.qattn_pool_last_l2(None, FAKE, 1024, 1024, cu.ctypes.data, 1, FAKE, 1024, None) == qattn.EINVAL
    assert b"NULL" in lib.qattn_last_error(None)
    assert lib.qattn_q4_matmul(None, FAKE, 64, 4, 64, FAKE, 2560, 8, FAKE, 8, None) == qattn.EINVAL
    assert lib.qattn_q4_matmul_swiglu(None, FAKE, 64, 4, 64, FAKE, 5120, 64, FAKE, 64, None) == qattn.EINVAL
    assert b"NULL" in lib.qattn_last_error(None)
