"""Pins the CPU oracle (oracle/pf_oracle.c) before the GPU path is tested against it.

Each check is chosen so that a plausible mistake fails it: closed-form offset
KATs (a wrong stride or a transposed block/segment index), the reference's
error rules, the merge-count closed form (1 + number of consecutive breaks),
an independent numpy brute force that addresses the layer tensor through a
strided array view, and the committed golden fixtures.  A planted-mistake
section shows that the golden data rejects the likely errors.
"""

import hashlib
import json
import os

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

import oracle
from oracle import OracleError

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

LLAMA = dict(nb=20000, bpb=32768)  # [2, 20000, 16, 8, 128] bf16


def llama_reg():
    kv = LLAMA["nb"] * LLAMA["bpb"]
    return oracle.layout(0x1000, 2 * kv, LLAMA["nb"], LLAMA["bpb"], kv, 2)


# ---------------------------------------------------------------------------
# Layout validation (lib.rs:389-449) and segment_offset (transfer.rs:18-47).
# ---------------------------------------------------------------------------
def test_llama_layout_closed_form():
    reg = llama_reg()
    assert reg.size_bytes == 1_310_720_000
    assert reg.block_size_bytes == 65_536
    assert reg.kv_stride_bytes == 655_360_000
    # V segment of block b sits at b*32768 + kv_stride.
    for b in (0, 1, 7, 19999):
        assert oracle.segment_offset(reg, b, 0) == b * 32768
        assert oracle.segment_offset(reg, b, 1) == b * 32768 + 655_360_000
    assert oracle.layout_kind(reg) == oracle.SPLIT
    assert not oracle.is_contiguous(reg)


@pytest.mark.parametrize(
    "args,msg",
    [
        ((0, 100, 10, 0, 10, 2), "invalid KV cache layout"),
        ((0, 100, 0, 10, 10, 2), "invalid KV cache layout"),
        ((0, 100, 10, 10, 10, 0), "invalid KV cache layout"),
        ((0, 1000, 10, 10, 0, 2), "kv_stride_bytes must be > 0"),
        ((0, 199, 10, 10, 100, 2), "registered memory too small"),
        ((0, 2**64 - 1, 2**63, 4, 0, 1), "num_blocks"),
        ((0, 2**64 - 1, 2, 2**63, 2**63, 2), "overflow"),
    ],
)
def test_layout_errors(args, msg):
    with pytest.raises(OracleError, match=msg):
        oracle.layout(*args)


def test_layout_exact_fit_accepted():
    # end = (nb-1)*bpb + (segments-1)*stride + bpb must be <= size (equality ok).
    reg = oracle.layout(0, 200, 10, 10, 100, 2)
    assert reg.block_size_bytes == 20
    with pytest.raises(OracleError):
        oracle.layout(0, 199, 10, 10, 100, 2)


def test_segment_offset_errors():
    reg = oracle.layout(0, 200, 10, 10, 100, 2)
    with pytest.raises(OracleError, match="Segment index out of range"):
        oracle.segment_offset(reg, 0, 2)
    assert oracle.segment_offset(reg, 9, 1) == 190
    # A block past num_blocks is only caught by the size bound.
    with pytest.raises(OracleError, match="Block 10 segment 1 exceeds registered memory"):
        oracle.segment_offset(reg, 10, 1)
    assert oracle.segment_offset(reg, 10, 0) == 100  # bound check only: in range
    with pytest.raises(OracleError, match="Block offset overflow"):
        oracle.segment_offset(reg, 2**62, 0)


def test_layout_kinds():
    assert oracle.layout_kind(oracle.layout(0, 200, 10, 10, 100, 2)) == oracle.SPLIT
    assert oracle.layout_kind(oracle.layout(0, 100, 10, 10, 0, 1)) == oracle.CONTIGUOUS
    # kv_stride == bytes_per_block counts as contiguous (transfer.rs:50-52).
    assert oracle.layout_kind(oracle.layout(0, 110, 10, 10, 10, 2)) == oracle.CONTIGUOUS
    # kv_stride < bytes_per_block and 3-segment layouts are neither.
    assert oracle.layout_kind(oracle.layout(0, 200, 10, 10, 5, 2)) == oracle.STRIDED
    assert oracle.layout_kind(oracle.layout(0, 400, 10, 10, 100, 3)) == oracle.STRIDED


# ---------------------------------------------------------------------------
# Run merging (transfer.rs:134-177).
# ---------------------------------------------------------------------------
def merge_count_closed_form(g, c, seg):
    if len(g) == 0:
        return 0
    breaks = sum(1 for j in range(1, len(g))
                 if not (g[j] == g[j - 1] + seg and c[j] == c[j - 1] + seg))
    return 1 + breaks


@settings(max_examples=200, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 6), st.integers(0, 6)), max_size=40),
       st.sampled_from([1, 16, 4096]))
def test_merge_runs_closed_form(steps, seg):
    # Build offsets by walking: a step of 1 continues the run on that side.
    g, c = [], []
    x, y = 1000 * seg, 5000 * seg
    for dg, dc in steps:
        x += dg * seg
        y += dc * seg
        g.append(x)
        c.append(y)
    runs = oracle.merge_runs(g, c, seg)
    assert len(runs) == merge_count_closed_form(g, c, seg)
    # Runs partition the list in order, and each satisfies the predicate.
    pos = 0
    for start, count in runs:
        assert start == pos and count >= 1
        for k in range(count):
            assert g[start + k] == g[start] + k * seg
            assert c[start + k] == c[start] + k * seg
        pos += count
    assert pos == len(g)


def test_merge_runs_cases():
    seg = 32768
    ids = np.arange(64)
    # Sorted consecutive ids with a packed host region: one copy.
    assert len(oracle.merge_runs(ids * seg, 10**9 + ids * seg, seg)) == 1
    # Device-contiguous but host-reversed: no merge.
    assert len(oracle.merge_runs(ids * seg, 10**9 + ids[::-1] * seg, seg)) == 64
    # Random ids (no adjacent pairs) defeat merging.
    rng = np.random.default_rng(0)
    r = rng.choice(20000, 640, replace=False)
    expect = merge_count_closed_form(list(r * seg), list(10**9 + np.arange(640) * seg), seg)
    assert len(oracle.merge_runs(r * seg, 10**9 + np.arange(640) * seg, seg)) == expect
    assert oracle.merge_runs([], [], seg) == []


# ---------------------------------------------------------------------------
# Save / load planning (lib.rs:590-705, 1032-1043).
# ---------------------------------------------------------------------------
def test_plan_save_filters():
    reg = oracle.layout(0, 200, 10, 10, 100, 2)
    assert list(oracle.plan_save(reg, [3, -1, 5, -7, 0])) == [3, 5, 0]
    assert list(oracle.plan_save(reg, [3, 4, 5], skip=[0, 1, 0])) == [3, 5]
    with pytest.raises(OracleError, match="block 10 out of range"):
        oracle.plan_save(reg, [3, 10])
    # Out-of-range is reported even for an entry that would be skipped.
    with pytest.raises(OracleError, match="out of range"):
        oracle.plan_save(reg, [11], skip=[1])


def test_save_host_layout():
    reg = oracle.layout(0, 200, 10, 10, 100, 2)
    k, v, split = oracle.save_host_layout(reg, 3, 1000, 5000)
    assert split and list(k) == [1000, 1010, 1020] and list(v) == [5000, 5010, 5020]
    reg1 = oracle.layout(0, 100, 10, 10, 0, 1)
    k, v, split = oracle.save_host_layout(reg1, 3, 1000, 0)
    assert not split and list(k) == [1000, 1010, 1020] and list(v) == [0, 0, 0]


def test_plan_load_filters():
    assert list(oracle.plan_load([4, -1, 2, 9], present=[1, 1, 0, 1])) == [0, 3]
    assert list(oracle.plan_load([-2, -1])) == []


# ---------------------------------------------------------------------------
# Bytes: oracle vs an independent strided-view brute force.
# ---------------------------------------------------------------------------
def strided(buf, reg):
    return np.lib.stride_tricks.as_strided(
        buf, shape=(int(reg.segments), int(reg.num_blocks), int(reg.bytes_per_block)),
        strides=(int(reg.kv_stride_bytes), int(reg.bytes_per_block), 1), writeable=True)


def brute_save_split(buf, reg, kept):
    v = strided(buf, reg)
    return (np.concatenate([v[0, b] for b in kept]), np.concatenate([v[1, b] for b in kept]))


layouts = st.one_of(
    # KV-first split, possibly padded between K and V.
    st.tuples(st.integers(2, 24), st.sampled_from([8, 16, 48, 64]), st.integers(0, 3),
              st.just(2)),
    # Single segment (blocks-first / MLA).
    st.tuples(st.integers(2, 24), st.sampled_from([8, 16, 48, 64]), st.just(0), st.just(1)),
)


@settings(max_examples=150, deadline=None)
@given(layouts, st.data())
def test_save_load_vs_bruteforce(lay, data):
    nb, bpb, pad_blocks, segments = lay
    kv = (nb + pad_blocks) * bpb if segments == 2 else 0
    size = kv + nb * bpb if segments == 2 else nb * bpb
    buf = np.random.default_rng(nb * 131 + bpb).integers(0, 256, size, dtype=np.uint8)
    reg = oracle.layout(buf.ctypes.data, size, nb, bpb, kv, segments)
    n = data.draw(st.integers(1, nb))
    ids = data.draw(st.lists(st.integers(-2, nb - 1), min_size=n, max_size=n))
    kept = [b for b in ids if b >= 0]
    plan = oracle.plan_save(reg, ids)
    assert list(plan) == kept
    if not kept:
        return
    m = len(kept)
    bs = int(reg.block_size_bytes)
    host = np.zeros(2 * m * bs, np.uint8)
    base = host.ctypes.data
    k_dst, v_dst, split = oracle.save_host_layout(reg, m, base, base + m * bpb)
    orig = buf.copy()
    oracle.process_save(reg, buf, plan, k_dst, v_dst)
    assert np.array_equal(buf, orig)  # save never writes the source
    if split:
        kr, vr = brute_save_split(orig, reg, kept)
        assert np.array_equal(host[: m * bpb], kr)
        assert np.array_equal(host[m * bpb: 2 * m * bpb], vr)
    else:
        blocks = orig.reshape(nb, bs)
        assert np.array_equal(host[: m * bs], np.concatenate([blocks[b] for b in kept]))
    # Load into targets: a permutation of distinct blocks.
    targets = data.draw(st.permutations(range(nb)))[:m]
    n_copies = oracle.process_load(reg, buf, np.array(targets), k_dst, v_dst)
    assert n_copies >= 1
    expect = orig.copy()
    if split:
        ev = strided(expect, reg)
        ov = strided(orig, reg)
        for j, b in enumerate(targets):
            ev[0, b] = ov[0, kept[j]]
            ev[1, b] = ov[1, kept[j]]
    else:
        eb, ob = expect.reshape(nb, bs), orig.reshape(nb, bs)
        for j, b in enumerate(targets):
            eb[b] = ob[kept[j]]
    assert np.array_equal(buf, expect)
    # Untouched blocks unchanged, including the padding between K and V.
    touched = np.zeros(size, bool)
    for b in targets:
        for s in range(segments):
            o = s * kv + b * bpb
            touched[o:o + bpb] = True
    assert np.array_equal(buf[~touched], orig[~touched])


def test_strided_layout_reference_behaviour():
    # segments == 2 with kv_stride < bytes_per_block: the reference saves each
    # segment separately (transfer.rs:217-239) but loads the whole block from
    # segment_offset(b, 0) (gpu_worker.rs:260-282).
    nb, bpb, stride = 6, 16, 8
    size = (nb - 1) * bpb + stride + bpb
    buf = np.arange(size, dtype=np.uint8)
    reg = oracle.layout(buf.ctypes.data, size, nb, bpb, stride, 2)
    assert oracle.layout_kind(reg) == oracle.STRIDED
    host = np.zeros(64, np.uint8)
    k_dst, _, _ = oracle.save_host_layout(reg, 1, host.ctypes.data, 0)
    oracle.process_save(reg, buf, [2], k_dst)
    assert np.array_equal(host[:16], buf[32:48])        # segment 0 of block 2
    assert np.array_equal(host[16:32], buf[40:56])      # segment 1 of block 2
    orig = buf.copy()
    oracle.process_load(reg, buf, [1], k_dst)
    assert np.array_equal(buf[16:48], host[:32])        # whole block at offset(1, 0)
    assert np.array_equal(buf[:16], orig[:16]) and np.array_equal(buf[48:], orig[48:])
    # The last block's whole-block load would run past the tensor: an error.
    with pytest.raises(OracleError, match="exceeds registered memory"):
        oracle.process_load(reg, buf, [nb - 1], k_dst)


def test_load_merges_like_reference():
    # Sorted consecutive targets with packed host regions: one copy for K and
    # one for V (transfer.rs:116-198 merges the two lists separately).
    nb, bpb = 16, 32
    kv = nb * bpb
    buf = np.zeros(2 * kv, np.uint8)
    reg = oracle.layout(buf.ctypes.data, 2 * kv, nb, bpb, kv, 2)
    host = np.arange(8 * bpb, dtype=np.uint8)
    base = host.ctypes.data
    k, v, _ = oracle.save_host_layout(reg, 4, base, base + 4 * bpb)
    assert oracle.process_load(reg, buf, [3, 4, 5, 6], k, v) == 2
    # K run end and V run start are contiguous on both sides only if the
    # lists merged across the K/V boundary; the reference never does that.
    assert oracle.process_load(reg, buf, [3, 5, 4, 6], k, v) == 8


# ---------------------------------------------------------------------------
# Golden fixtures.
# ---------------------------------------------------------------------------
def _run_fixture_split(f, layer):
    buf = f[f"input_{layer}"].copy()
    nb, bpb = int(f["num_blocks"]), int(f["bytes_per_block"])
    reg = oracle.layout(buf.ctypes.data, int(f["size_bytes"]), nb, bpb,
                        int(f["kv_stride_bytes"]), int(f["segments"]))
    plan = oracle.plan_save(reg, f["save_ids"])
    m = len(plan)
    host = np.zeros(2 * m * int(reg.block_size_bytes), np.uint8)
    k, v, split = oracle.save_host_layout(reg, m, host.ctypes.data,
                                          host.ctypes.data + m * bpb)
    oracle.process_save(reg, buf, plan, k, v)
    targets = oracle.plan_load(f["load_ids"])
    oracle.process_load(reg, buf, np.asarray(f["load_ids"])[targets], k, v)
    return host, buf, m, split


def test_golden_tiny_kvfirst():
    f = np.load(os.path.join(GOLDEN, "tiny_kvfirst.npz"))
    for layer in range(2):
        host, buf, m, split = _run_fixture_split(f, layer)
        bpb = int(f["bytes_per_block"])
        assert split
        assert np.array_equal(host[: m * bpb], f[f"host_k_{layer}"])
        assert np.array_equal(host[m * bpb: 2 * m * bpb], f[f"host_v_{layer}"])
        assert np.array_equal(buf, f[f"restored_{layer}"])


def test_golden_tiny_blocks():
    f = np.load(os.path.join(GOLDEN, "tiny_blocks.npz"))
    for layer in range(2):
        host, buf, m, split = _run_fixture_split(f, layer)
        assert not split
        assert np.array_equal(host[: m * int(f["bytes_per_block"])], f[f"host_{layer}"])
        assert np.array_equal(buf, f[f"restored_{layer}"])


def test_golden_gpt2_config1():
    """Config 1 (GPT-2 shape, the reference's CPU memcpy path): the oracle
    reproduces every committed digest."""
    with open(os.path.join(GOLDEN, "gpt2_config1.json")) as fh:
        g = json.load(fh)
    nb, bpb, kv = g["num_blocks"], g["bytes_per_block"], g["kv_stride_bytes"]
    m = len(g["save_ids"])
    host = np.zeros(2 * m * bpb, np.uint8)
    for layer in range(g["layers"]):
        buf = np.zeros(g["size_bytes"], np.uint8)
        oracle.fill_random(buf, oracle.layer_seed(g["base_seed"], layer))
        reg = oracle.layout(buf.ctypes.data, g["size_bytes"], nb, bpb, kv, 2)
        plan = oracle.plan_save(reg, g["save_ids"])
        k, v, _ = oracle.save_host_layout(reg, m, host.ctypes.data, host.ctypes.data + m * bpb)
        oracle.process_save(reg, buf, plan, k, v)
        assert hashlib.sha256(host[: m * bpb].tobytes()).hexdigest() == g["host_k_sha256"][layer]
        assert hashlib.sha256(host[m * bpb:].tobytes()).hexdigest() == g["host_v_sha256"][layer]
        oracle.process_load(reg, buf, g["load_ids"], k, v)
        assert hashlib.sha256(buf.tobytes()).hexdigest() == g["restored_sha256"][layer]


def test_fill_random_c_matches_numpy():
    buf = np.zeros(4096, np.uint8)
    oracle.fill_random(buf, 12345, word_offset=77)
    assert np.array_equal(buf.view(np.uint64), oracle.random_words(512, 12345, 77))
    # splitmix64 known answer: first output of the stream seeded with 0.
    assert int(oracle.random_words(1, 0)[0]) == 0xE220A8397B1DCDAF


# ---------------------------------------------------------------------------
# Planted mistakes: the fixtures reject them.
# ---------------------------------------------------------------------------
def test_planted_mistakes_are_caught():
    f = np.load(os.path.join(GOLDEN, "tiny_kvfirst.npz"))
    buf = f["input_0"].copy()
    nb, bpb, kv = int(f["num_blocks"]), int(f["bytes_per_block"]), int(f["kv_stride_bytes"])
    kept = [int(b) for b in f["save_ids"] if b >= 0]

    def save_with(offset_fn):
        return np.concatenate([buf[offset_fn(b, 0): offset_fn(b, 0) + bpb] for b in kept])

    good = save_with(lambda b, s: b * bpb + s * kv)
    assert np.array_equal(good, f["host_k_0"])
    mistakes = {
        "transposed index": lambda b, s: s * bpb + b * kv % len(buf),
        "stride off by one block": lambda b, s: (b + 1) * bpb + s * kv,
        "V instead of K": lambda b, s: b * bpb + (1 - s) * kv,
    }
    for name, fn in mistakes.items():
        got = save_with(fn)
        assert not np.array_equal(got, f["host_k_0"]), name
    # Keeping a negative id (a dropped filter) changes the host region length.
    assert len(f["host_k_0"]) == len(kept) * bpb != len(f["save_ids"]) * bpb
