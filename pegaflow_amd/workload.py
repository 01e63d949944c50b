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


def verify_saved(layers: DeviceLayers, saved: list[LayerTransfer]) -> int:
    """Mismatching words in the host regions of a save batch (0 = exact)."""
    bad = 0
    for l, lt in enumerate(saved):
        reg = lt.registration
        ids = lt.blocks["block_idx"].astype(np.uint64)
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
    shape = layers.shape
    nb, bpb = shape.num_blocks, shape.bytes_per_block
    blocks = np.arange(nb, dtype=np.uint64)
    src = blocks.copy()
    src[np.asarray(targets, np.int64)] = np.asarray(ids, np.uint64)
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
           "DeviceLayers", "save_plan", "load_plan", "verify_saved", "verify_restored",
           "layer_seed", "payload_bytes", "MiB", "_lib"]
