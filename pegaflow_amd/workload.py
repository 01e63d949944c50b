"""Synthetic KV workloads for benchmarks and checks: layer tensors filled with
seeded random bits on the device, block-id draws, the reference's host block
layout for a save batch, and closed-form verification on the device.

Contents are splitmix64 words: word i of a layer tensor is
mix64(seed_l + (i + 1) * 0x9E3779B97F4A7C15), so the expected bytes of any
block are known without keeping a copy, and a save/restore can be checked at
full size by the device verify kernel.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, verify_random_chunks
from .transfer import BLOCK_DTYPE, KVCacheRegistration, LayerTransfer

MiB = 1 << 20


def layer_seed(base_seed: int, layer: int) -> int:
    return (base_seed * 0x100000001B3 + layer * 0xD1B54A32D192ED03 + 1) % 2**64


@dataclass(frozen=True)
class KVShape:
    """Per-layer paged KV tensor: KV-first [2, num_blocks, tokens, heads, dim]
    (segments=2) or blocks-first [num_blocks, tokens, latent] (segments=1)."""

    name: str
    layers: int
    num_blocks: int
    bytes_per_block: int
    segments: int

    @property
    def kv_stride_bytes(self) -> int:
        return self.num_blocks * self.bytes_per_block if self.segments == 2 else 0

    @property
    def layer_bytes(self) -> int:
        return self.num_blocks * self.bytes_per_block * self.segments


# The workloads of the transfer-path benchmark (block = 16 tokens unless noted).
GPT2 = KVShape("gpt2 fp16 [2,512,16,12,64]", 12, 512, 16 * 12 * 64 * 2, 2)
LLAMA3_8B = KVShape("llama-3.1-8b bf16 [2,20000,16,8,128]", 32, 20000, 16 * 8 * 128 * 2, 2)
QWEN3_8B = KVShape("qwen3-8b bf16 [2,16000,16,8,128]", 36, 16000, 16 * 8 * 128 * 2, 2)
# One tensor-parallel rank of Llama-3.1-8B at TP=8: one kv head, 4 KiB segments.
LLAMA3_8B_TP8_RANK = KVShape("llama-3.1-8b tp8 rank bf16 [2,20000,16,1,128]", 32, 20000,
                             16 * 1 * 128 * 2, 2)
MLA_BF16 = KVShape("mla-latent bf16 [8192,64,576]", 61, 8192, 64 * 576 * 2, 1)
MLA_FP8 = KVShape("mla-latent fp8 [8192,64,576]", 61, 8192, 64 * 576, 1)


def draw_blocks(num_blocks: int, n: int, seed: int = 0):
    """(save ids, load targets): n distinct ids drawn uniformly in draw order,
    and n other distinct ids for the restore."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ids = rng.choice(num_blocks, n, replace=False)
    rest = np.setdiff1d(np.arange(num_blocks), ids)
    targets = rng.choice(rest, n, replace=False)
    return ids.astype(np.int64), targets.astype(np.int64)


def draw_runs(rng, num_blocks: int, n: int, mean_run: float, exclude=None) -> np.ndarray:
    """n distinct block ids built from runs of consecutive blocks whose
    lengths are Geometric(1/mean_run) (support >= 1), each run starting at a
    random free block and stopping early at a used block or the tensor's end.
    mean_run >= n gives one sorted consecutive run at a random free window.
    ``exclude``: a bool mask of num_blocks blocks that may not be drawn.
    Ids are returned in draw order (the reference never sorts)."""
    used = np.zeros(num_blocks, bool) if exclude is None else np.array(exclude, bool)
    if used.shape != (num_blocks,):
        raise ValueError("exclude must be a mask of num_blocks entries")
    if n > num_blocks - int(used.sum()):
        raise ValueError(f"cannot draw {n} distinct blocks: {num_blocks - int(used.sum())} free")
    if mean_run >= n:
        # Start positions s whose window [s, s + n) holds no used block.
        c = np.concatenate([[0], np.cumsum(used, dtype=np.int64)])
        starts = np.flatnonzero(c[n:] - c[:-n] == 0)
        if len(starts) == 0:
            raise ValueError(f"no free window of {n} consecutive blocks")
        s = int(starts[int(rng.integers(0, len(starts)))])
        return np.arange(s, s + n, dtype=np.int64)
    out = []
    while len(out) < n:
        length = min(int(rng.geometric(1.0 / mean_run)), n - len(out))
        b = int(rng.integers(0, num_blocks))
        while used[b]:
            b = int(rng.integers(0, num_blocks))
        while length > 0 and b < num_blocks and not used[b]:
            used[b] = True
            out.append(b)
            b += 1
            length -= 1
    return np.asarray(out, np.int64)


def run_count(ids) -> int:
    """Maximal runs of consecutive increasing ids (1 + breaks)."""
    ids = np.asarray(ids, np.int64)
    return 0 if len(ids) == 0 else 1 + int(np.count_nonzero(np.diff(ids) != 1))


def fragmentation_requests(num_blocks: int, mean_run: float, seed: int = 0,
                           n_requests: int = 64, min_tokens: int = 1024,
                           max_tokens: int = 16384, block_tokens: int = 16):
    """The fragmentation sweep's batch: n_requests prefixes of U[min_tokens,
    max_tokens] tokens (ceil(tokens / block_tokens) blocks each).  Each
    request is (ids, targets): the blocks it saves, drawn as geometric runs
    of mean ``mean_run``, and the blocks it restores that batch into, a
    second draw of the same kind disjoint from ``ids``.  Each request saves
    and then restores the same bytes, so saves and restores alternate 50/50.
    mean_run >= SORTED_MEAN_RUN (640, the 10K-token prefix's block count)
    stands for fully sorted ids: one consecutive run per request, whatever
    its length.  The same seed gives the same token counts for every
    mean_run."""
    tok_rng = np.random.Generator(np.random.PCG64(seed + 4))
    tokens = tok_rng.integers(min_tokens, max_tokens + 1, n_requests)
    rng = np.random.Generator(np.random.PCG64([seed + 4, int(round(mean_run * 1000))]))
    m = float("inf") if mean_run >= SORTED_MEAN_RUN else mean_run
    out = []
    for t in tokens:
        nb = (int(t) + block_tokens - 1) // block_tokens
        ids = draw_runs(rng, num_blocks, nb, m)
        mask = np.zeros(num_blocks, bool)
        mask[ids] = True
        out.append((ids, draw_runs(rng, num_blocks, nb, m, exclude=mask)))
    return out


SORTED_MEAN_RUN = 640


class DeviceLayers:
    """One device tensor per layer, filled with seeded random words."""

    def __init__(self, shape: KVShape, base_seed: int = 0, layers: int | None = None):
        self.shape = shape
        n = shape.layers if layers is None else layers
        self.seeds = [layer_seed(base_seed, l) for l in range(n)]
        self.bufs = [DeviceBuffer(shape.layer_bytes) for _ in range(n)]
        self.regs = [KVCacheRegistration.create(b.ptr, shape.layer_bytes, shape.num_blocks,
                                                shape.bytes_per_block, shape.kv_stride_bytes,
                                                shape.segments) for b in self.bufs]
        self.refill()

    def refill(self) -> None:
        for b, s in zip(self.bufs, self.seeds):
            b.fill_random(s)

    def close(self) -> None:
        for b in self.bufs:
            b.close()
        self.bufs = []


def save_plan(regs, ids, host_base: int) -> list[LayerTransfer]:
    """A save batch in the reference's host layout (lib.rs:636-747), one
    layer after another from host_base: split layers get a K region then a V
    region (block i at i*bytes_per_block in each); other layers one region of
    whole blocks (block i at i*block_size_bytes)."""
    ids = np.asarray(ids, np.int64)
    n = len(ids)
    out, base = [], host_base
    for reg in regs:
        blocks = np.zeros(n, BLOCK_DTYPE)
        blocks["block_idx"] = ids
        if reg.is_split:
            seg = reg.bytes_per_block
            blocks["k_host"] = base + np.arange(n, dtype=np.uint64) * seg
            blocks["v_host"] = base + n * seg + np.arange(n, dtype=np.uint64) * seg
        else:
            blocks["k_host"] = base + np.arange(n, dtype=np.uint64) * reg.block_size_bytes
        out.append(LayerTransfer(reg, blocks))
        base += n * reg.block_size_bytes
    return out


def load_plan(saved: list[LayerTransfer], targets) -> list[LayerTransfer]:
    """The restore of a saved batch into other blocks (same host sources)."""
    out = []
    for lt in saved:
        b = lt.blocks.copy()
        b["block_idx"] = np.asarray(targets, np.int64)
        out.append(LayerTransfer(lt.registration, b))
    return out


def verify_saved(layers: DeviceLayers, saved: list[LayerTransfer], src_of=None) -> int:
    """Mismatching words in the host regions of a save batch (0 = exact).
    ``src_of`` (optional, one entry per block): block b currently holds the
    words block src_of[b] was filled with (after earlier restores)."""
    bad = 0
    for l, lt in enumerate(saved):
        reg = lt.registration
        ids = lt.blocks["block_idx"].astype(np.uint64)
        if src_of is not None:
            ids = np.asarray(src_of, np.uint64)[ids.astype(np.int64)]
        bpb = reg.bytes_per_block
        if reg.is_split:
            addrs = np.concatenate([lt.blocks["k_host"], lt.blocks["v_host"]])
            offs = np.concatenate([ids * bpb // 8, (reg.kv_stride_bytes + ids * bpb) // 8])
            bad += verify_random_chunks(addrs, offs, bpb, layers.seeds[l])
        else:
            bad += verify_random_chunks(lt.blocks["k_host"], ids * bpb // 8,
                                        reg.block_size_bytes, layers.seeds[l])
    return bad


def verify_restored(layers: DeviceLayers, ids, targets) -> int:
    """Mismatching words over every block of every layer after restoring the
    blocks saved from `ids` into `targets` (0 = exact, untouched blocks
    included)."""
    src = np.arange(layers.shape.num_blocks, dtype=np.uint64)
    src[np.asarray(targets, np.int64)] = np.asarray(ids, np.uint64)
    return verify_blocks(layers, src)


def verify_blocks(layers: DeviceLayers, src_of) -> int:
    """Mismatching words over every block of every layer: block b must hold
    the words block src_of[b] was filled with (0 = exact)."""
    shape = layers.shape
    nb, bpb = shape.num_blocks, shape.bytes_per_block
    blocks = np.arange(nb, dtype=np.uint64)
    src = np.asarray(src_of, np.uint64)
    if src.shape != (nb,):
        raise ValueError("src_of needs one entry per block")
    bad = 0
    for l, buf in enumerate(layers.bufs):
        if shape.segments == 2:
            addrs = np.concatenate([buf.ptr + blocks * bpb,
                                    buf.ptr + shape.kv_stride_bytes + blocks * bpb])
            offs = np.concatenate([src * bpb // 8, (shape.kv_stride_bytes + src * bpb) // 8])
        else:
            addrs = buf.ptr + blocks * bpb
            offs = src * bpb // 8
        bad += verify_random_chunks(addrs, offs, bpb, layers.seeds[l])
    return bad


def payload_bytes(regs, n_blocks: int) -> int:
    return sum(n_blocks * r.block_size_bytes for r in regs)


__all__ = ["KVShape", "GPT2", "LLAMA3_8B", "LLAMA3_8B_TP8_RANK", "QWEN3_8B", "MLA_BF16", "MLA_FP8", "draw_blocks",
           "draw_runs", "run_count", "fragmentation_requests",
           "DeviceLayers", "save_plan", "load_plan", "verify_saved", "verify_restored",
           "verify_blocks", "layer_seed", "payload_bytes", "MiB", "_lib"]
