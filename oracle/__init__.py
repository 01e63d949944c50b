"""CPU oracle for PegaFlow's KV-block transfer path.

TEST INFRASTRUCTURE ONLY.  The HIP product path (``pegaflow_amd``) is tested
against this package, and it is the CPU baseline timed beside it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import
it; the product never does.

The arithmetic lives in ``pf_oracle.c`` (a restatement of the reference's
``pegaflow-core/src/transfer.rs``, ``gpu_worker.rs:205-390`` and the planning
parts of ``lib.rs``); this module is a ctypes wrapper plus the synthetic-data
generator shared with the tests.

Parity pinning (see tests/test_oracle.py):
  * segment offsets and layout validation: closed-form integer KATs and
    hand-built edge cases (transfer.rs:18-47, lib.rs:389-449);
  * run merging: the number of runs equals 1 + the number of consecutive
    breaks of the merge predicate, checked on random and hand-built lists;
  * save / load bytes: an independent numpy brute force that indexes the
    layer tensor as an array ``[segments, num_blocks, ...]`` instead of byte
    offsets, plus the permutation identity and "untouched blocks unchanged";
  * committed golden digests for the GPT-2-shape workload (tests/golden/).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

GOLDEN_GAMMA = 0x9E3779B97F4A7C15

SPLIT, CONTIGUOUS, STRIDED = 0, 1, 2


class OracleError(RuntimeError):
    pass


class Layout(ctypes.Structure):
    """KVCacheRegistration (lib.rs:100-112)."""

    _fields_ = [
        ("data_ptr", ctypes.c_uint64),
        ("size_bytes", ctypes.c_uint64),
        ("num_blocks", ctypes.c_uint64),
        ("bytes_per_block", ctypes.c_uint64),
        ("block_size_bytes", ctypes.c_uint64),
        ("kv_stride_bytes", ctypes.c_uint64),
        ("segments", ctypes.c_uint64),
    ]


def build() -> str:
    """Compile liboracle.so with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u64, p64 = ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)
        pl = ctypes.POINTER(Layout)
        cp, sz = ctypes.c_char_p, ctypes.c_size_t
        L.or_layout_init.argtypes = [u64] * 6 + [pl, cp, sz]
        L.or_segment_offset.argtypes = [pl, u64, u64, p64, cp, sz]
        L.or_is_contiguous.argtypes = [pl]
        L.or_layout_kind.argtypes = [pl]
        L.or_merge_runs.argtypes = [p64, p64, u64, u64, p64, p64]
        L.or_merge_runs.restype = u64
        L.or_plan_save.argtypes = [pl, ctypes.c_void_p, u64, ctypes.c_void_p,
                                   ctypes.c_void_p, p64, cp, sz]
        L.or_save_host_layout.argtypes = [pl, u64, u64, u64, p64, p64]
        L.or_plan_load.argtypes = [ctypes.c_void_p, ctypes.c_void_p, u64, p64]
        L.or_plan_load.restype = u64
        for fn in (L.or_save_copies, L.or_load_copies):
            fn.argtypes = [pl, u64, ctypes.c_void_p, p64, p64, u64, p64, p64,
                           p64, cp, sz]
            fn.restype = u64
        L.or_run_copies.argtypes = [p64, p64, p64, u64, ctypes.c_int]
        L.or_process_save.argtypes = [pl, u64, ctypes.c_void_p, p64, p64, u64,
                                      cp, sz]
        L.or_process_load.argtypes = [pl, u64, ctypes.c_void_p, p64, p64, u64,
                                      p64, cp, sz]
        L.or_fill_random.argtypes = [u64, u64, u64, u64]
        L.or_pack_blocks.argtypes = [u64, u64, p64, p64, p64, u64, p64]
        L.or_pack_blocks.restype = u64
        L.or_unpack_block.argtypes = [u64, u64, ctypes.c_void_p, p64, p64, p64]
        _lib = L
    return _lib


def _p64(a: np.ndarray):
    assert a.dtype == np.uint64 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))


def _err():
    return ctypes.create_string_buffer(512)


def layout(data_ptr, size_bytes, num_blocks, bytes_per_block, kv_stride_bytes,
           segments) -> Layout:
    """register_context_layer validation (lib.rs:389-449)."""
    out, err = Layout(), _err()
    rc = lib().or_layout_init(data_ptr, size_bytes, num_blocks, bytes_per_block,
                              kv_stride_bytes, segments, ctypes.byref(out),
                              err, 512)
    if rc:
        raise OracleError(err.value.decode())
    return out


def segment_offset(reg: Layout, block_idx: int, segment_idx: int) -> int:
    """transfer.rs:18-47."""
    out, err = ctypes.c_uint64(), _err()
    if lib().or_segment_offset(ctypes.byref(reg), block_idx, segment_idx,
                               ctypes.byref(out), err, 512):
        raise OracleError(err.value.decode())
    return out.value


def is_contiguous(reg: Layout) -> bool:
    return bool(lib().or_is_contiguous(ctypes.byref(reg)))


def layout_kind(reg: Layout) -> int:
    return lib().or_layout_kind(ctypes.byref(reg))


def merge_runs(gpu_off, cpu_addr, seg):
    """transfer.rs:134-177: list of (start, count)."""
    g = np.ascontiguousarray(gpu_off, dtype=np.uint64)
    c = np.ascontiguousarray(cpu_addr, dtype=np.uint64)
    n = len(g)
    rs = np.zeros(max(n, 1), np.uint64)
    rc = np.zeros(max(n, 1), np.uint64)
    runs = lib().or_merge_runs(_p64(g), _p64(c), n, seg, _p64(rs), _p64(rc))
    return [(int(rs[i]), int(rc[i])) for i in range(runs)]


def plan_save(reg: Layout, block_ids, skip=None) -> np.ndarray:
    """lib.rs:590-621: kept block indices (int64) in order."""
    ids = np.ascontiguousarray(block_ids, dtype=np.int32)
    sk = None if skip is None else np.ascontiguousarray(skip, dtype=np.uint8)
    out = np.zeros(max(len(ids), 1), np.int64)
    n_out, err = ctypes.c_uint64(), _err()
    if lib().or_plan_save(ctypes.byref(reg), ids.ctypes.data, len(ids),
                          None if sk is None else sk.ctypes.data,
                          out.ctypes.data, ctypes.byref(n_out), err, 512):
        raise OracleError(err.value.decode())
    return out[: n_out.value].copy()


def save_host_layout(reg: Layout, n: int, k_base: int, v_base: int):
    """lib.rs:636-747: per-block host destinations (k_dst, v_dst, split?)."""
    k = np.zeros(max(n, 1), np.uint64)
    v = np.zeros(max(n, 1), np.uint64)
    split = lib().or_save_host_layout(ctypes.byref(reg), n, k_base, v_base,
                                      _p64(k), _p64(v))
    return k[:n].copy(), v[:n].copy(), bool(split)


def plan_load(block_ids, present=None) -> np.ndarray:
    """lib.rs:1032-1043: positions of the entries that are loaded."""
    ids = np.ascontiguousarray(block_ids, dtype=np.int32)
    pr = None if present is None else np.ascontiguousarray(present, np.uint8)
    out = np.zeros(max(len(ids), 1), np.uint64)
    k = lib().or_plan_load(ids.ctypes.data, None if pr is None else pr.ctypes.data,
                           len(ids), _p64(out))
    return out[:k].copy()


def _copies(fn, reg, dev_addr, block_idx, k, v, cap):
    bi = np.ascontiguousarray(block_idx, dtype=np.int64)
    k = np.ascontiguousarray(k, dtype=np.uint64)
    v = np.zeros_like(k) if v is None else np.ascontiguousarray(v, np.uint64)
    src = np.zeros(max(cap, 1), np.uint64)
    dst = np.zeros(max(cap, 1), np.uint64)
    size = np.zeros(max(cap, 1), np.uint64)
    err = _err()
    c = fn(ctypes.byref(reg), dev_addr, bi.ctypes.data, _p64(k), _p64(v),
           len(bi), _p64(src), _p64(dst), _p64(size), err, 512)
    if c == 2**64 - 1:
        raise OracleError(err.value.decode())
    return src[:c].copy(), dst[:c].copy(), size[:c].copy()


def save_copies(reg, dev_addr, block_idx, k_dst, v_dst=None):
    """The cuMemcpyDtoH calls of one save task (gpu_worker.rs:321-372)."""
    cap = len(block_idx) * max(2, int(reg.segments))
    return _copies(lib().or_save_copies, reg, dev_addr, block_idx, k_dst,
                   v_dst, cap)


def load_copies(reg, dev_addr, block_idx, k_src, v_src=None):
    """The merged cuMemcpyHtoDAsync calls of one load layer
    (gpu_worker.rs:211-283, transfer.rs:116-198)."""
    return _copies(lib().or_load_copies, reg, dev_addr, block_idx, k_src,
                   v_src, 2 * len(block_idx))


def run_copies(src, dst, size, nthreads=1):
    src = np.ascontiguousarray(src, np.uint64)
    dst = np.ascontiguousarray(dst, np.uint64)
    size = np.ascontiguousarray(size, np.uint64)
    lib().or_run_copies(_p64(src), _p64(dst), _p64(size), len(src), nthreads)


def process_save(reg, dev: np.ndarray, block_idx, k_dst, v_dst=None):
    """Save task on host memory: dev is the host copy of the layer tensor."""
    src, dst, size = save_copies(reg, dev.ctypes.data, block_idx, k_dst, v_dst)
    run_copies(src, dst, size)


def process_load(reg, dev: np.ndarray, block_idx, k_src, v_src=None) -> int:
    """Load layer on host memory; returns the number of merged copies."""
    src, dst, size = load_copies(reg, dev.ctypes.data, block_idx, k_src, v_src)
    run_copies(src, dst, size)
    return len(src)


# --------------------------------------------------------------------------
# Synthetic contents shared by tests, smoke and bench: splitmix64 words.
# --------------------------------------------------------------------------
def mix64_np(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64, copy=True)
    z ^= z >> np.uint64(30)
    z *= np.uint64(0xBF58476D1CE4E5B9)
    z ^= z >> np.uint64(27)
    z *= np.uint64(0x94D049BB133111EB)
    z ^= z >> np.uint64(31)
    return z


def random_words(n_words: int, seed: int, word_offset: int = 0) -> np.ndarray:
    """word[i] = mix64(seed + (word_offset + i + 1) * GAMMA) (numpy)."""
    with np.errstate(over="ignore"):
        i = np.arange(word_offset + 1, word_offset + 1 + n_words, dtype=np.uint64)
        z = np.uint64(seed) + i * np.uint64(GOLDEN_GAMMA)
        return mix64_np(z)


def fill_random(buf: np.ndarray, seed: int, word_offset: int = 0) -> None:
    """C version of random_words, in place (size multiple of 8)."""
    assert buf.flags.c_contiguous and buf.nbytes % 8 == 0
    lib().or_fill_random(buf.ctypes.data, buf.nbytes, seed, word_offset)


def layer_seed(base_seed: int, layer: int) -> int:
    """Per-layer seed used by the synthetic workloads."""
    return (base_seed * 0x100000001B3 + layer * 0xD1B54A32D192ED03 + 1) % 2**64


# --------------------------------------------------------------------------
# Packed block files of the disk tier (seal_offload.rs).
# --------------------------------------------------------------------------
def pack_blocks(blocks) -> tuple[bytes, list[int]]:
    """write_packed_file (seal_offload.rs:379-448).  ``blocks`` is a list of
    blocks, each a list of slots (K bytes, V bytes or None).  Returns the
    file bytes and each block's offset."""
    n = len(blocks)
    s = len(blocks[0]) if n else 0
    keep = []
    k = np.zeros(max(n * s, 1), np.uint64)
    v = np.zeros(max(n * s, 1), np.uint64)
    size = np.zeros(max(n * s, 1), np.uint64)
    for b, slots in enumerate(blocks):
        assert len(slots) == s
        for j, (kb, vb) in enumerate(slots):
            ka = np.frombuffer(bytes(kb) or b"\0", np.uint8).copy()
            keep.append(ka)
            k[b * s + j] = ka.ctypes.data
            if vb is None:
                size[b * s + j] = len(kb)
            else:
                assert len(vb) == len(kb)
                va = np.frombuffer(bytes(vb) or b"\0", np.uint8).copy()
                keep.append(va)
                v[b * s + j] = va.ctypes.data
                size[b * s + j] = 2 * len(kb)
    offs = np.zeros(max(n, 1), np.uint64)
    total = lib().or_pack_blocks(n, s, _p64(k), _p64(v), _p64(size), 0, _p64(offs))
    out = np.zeros(max(total, 1), np.uint8)
    lib().or_pack_blocks(n, s, _p64(k), _p64(v), _p64(size), out.ctypes.data, _p64(offs))
    return out[:total].tobytes(), [int(o) for o in offs[:n]]


def unpack_block(data: bytes, slots) -> list[tuple[bytes, bytes | None]]:
    """rebuild_sealed_block (seal_offload.rs:869-909): ``slots`` is the
    BlockMeta slot list [(is_split, size)]; returns (K, V or None) per slot."""
    s = len(slots)
    buf = np.frombuffer(bytes(data) or b"\0", np.uint8).copy()
    split = np.array([1 if sp else 0 for sp, _ in slots] or [0], np.uint8)
    size = np.array([sz for _, sz in slots] or [0], np.uint64)
    k = np.zeros(max(s, 1), np.uint64)
    v = np.zeros(max(s, 1), np.uint64)
    lib().or_unpack_block(buf.ctypes.data, s, split.ctypes.data, _p64(size), _p64(k), _p64(v))
    out = []
    base = buf.ctypes.data
    for j, (sp, sz) in enumerate(slots):
        ko = int(k[j]) - base
        if sp:
            vo = int(v[j]) - base
            out.append((buf[ko:ko + sz // 2].tobytes(), buf[vo:vo + sz // 2].tobytes()))
        else:
            out.append((buf[ko:ko + sz].tobytes(), None))
    return out


def block_meta_json(file: str, offset: int, slots, total_slots: int) -> str:
    """BlockMeta as serde_json renders it (seal_offload.rs:80-97): compact,
    fields in declaration order."""
    body = ",".join('{"is_split":%s,"size":%d}' % ("true" if sp else "false", sz)
                    for sp, sz in slots)
    return '{"file":"%s","offset":%d,"slots":[%s],"total_slots":%d}' % (
        file, offset, body, total_slots)
