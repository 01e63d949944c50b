"""Writes the golden fixtures of the KV-block transfer path.

The expected outputs come from a numpy brute force that is independent of the
oracle's byte-offset arithmetic: each layer tensor is viewed as a strided
array ``[segments, num_blocks, bytes_per_block]`` (numpy computes every
address) and save/load are written as array indexing, following the
semantics of the reference:
  * save (lib.rs:590-705, gpu_worker.rs:321-372): negative ids are skipped;
    for the KV-first split layout the host holds one K region and one V region,
    block i of the kept list at offset i * bytes_per_block in each; for a
    single-segment layout one region with block i at i * block_size_bytes;
  * load (lib.rs:1032-1043, gpu_worker.rs:205-283): entry j of the host
    regions goes to block B[j] of the tensor.

Fixtures:
  tiny_kvfirst.npz  — 2 fp16 layers [2, 8, 2, 2, 4], full byte vectors
  tiny_blocks.npz   — 2 bf16 layers [6, 4, 8] (blocks-first, 1 segment)
  gpt2_config1.json — the GPT-2-shape workload (12 layers, [2,512,16,12,64]
                      fp16, 64 saved blocks, 64 load targets): block ids and
                      SHA-256 digests of every host region and restored layer.
  packed_tiny.npz   — packed block files of the disk tier (seal_offload.rs:
                      379-448): 2 layers x tp 2 KV-first fp16 [2, 8, 2, 2, 4]
                      layers (4 split slots) and 1 blocks-first layer (one
                      contiguous slot); the file is the array
                      [block, slot, K|V, bytes] flattened, with each block's
                      BlockMeta JSON.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GAMMA = 0x9E3779B97F4A7C15


def mix64(z: np.ndarray) -> np.ndarray:
    z = z.copy()
    z ^= z >> np.uint64(30)
    z *= np.uint64(0xBF58476D1CE4E5B9)
    z ^= z >> np.uint64(27)
    z *= np.uint64(0x94D049BB133111EB)
    z ^= z >> np.uint64(31)
    return z


def random_bytes(nbytes: int, seed: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(1, nbytes // 8 + 1, dtype=np.uint64)
        words = mix64(np.uint64(seed) + i * np.uint64(GAMMA))
    return words.view(np.uint8).copy()


def layer_seed(base_seed: int, layer: int) -> int:
    return (base_seed * 0x100000001B3 + layer * 0xD1B54A32D192ED03 + 1) % 2**64


def segment_view(buf: np.ndarray, num_blocks: int, bpb: int, kv_stride: int, segments: int):
    """[segments, num_blocks, bpb] byte view of a layer buffer."""
    return np.lib.stride_tricks.as_strided(
        buf, shape=(segments, num_blocks, bpb), strides=(kv_stride, bpb, 1), writeable=True)


def brute_save(buf, num_blocks, bpb, kv_stride, segments, block_ids):
    kept = [b for b in block_ids if b >= 0]
    v = segment_view(buf, num_blocks, bpb, kv_stride, segments)
    if segments == 2 and kv_stride > bpb:
        k_region = np.concatenate([v[0, b] for b in kept]) if kept else np.zeros(0, np.uint8)
        v_region = np.concatenate([v[1, b] for b in kept]) if kept else np.zeros(0, np.uint8)
        return kept, k_region, v_region
    blocks = np.lib.stride_tricks.as_strided(
        buf, shape=(num_blocks, bpb * segments), strides=(bpb, 1))
    region = np.concatenate([blocks[b] for b in kept]) if kept else np.zeros(0, np.uint8)
    return kept, region, None


def brute_load(buf, num_blocks, bpb, kv_stride, segments, targets, k_region, v_region):
    v = segment_view(buf, num_blocks, bpb, kv_stride, segments)
    if segments == 2 and kv_stride > bpb:
        for j, b in enumerate(targets):
            v[0, b] = k_region[j * bpb:(j + 1) * bpb]
            v[1, b] = v_region[j * bpb:(j + 1) * bpb]
        return
    bs = bpb * segments
    blocks = np.lib.stride_tricks.as_strided(buf, shape=(num_blocks, bs), strides=(bpb, 1),
                                             writeable=True)
    for j, b in enumerate(targets):
        blocks[b] = k_region[j * bs:(j + 1) * bs]


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def make_tiny_kvfirst():
    # [2, 8 blocks, 2 tokens, 2 heads, 4 dim] fp16: bpb = 32 B, kv_stride = 256 B.
    nb, bpb, layers = 8, 2 * 2 * 4 * 2, 2
    kv_stride = nb * bpb
    size = 2 * kv_stride
    save_ids = np.array([5, -1, 2, 7], np.int32)
    load_ids = np.array([1, 3, 0], np.int32)
    out = {"num_blocks": nb, "bytes_per_block": bpb, "kv_stride_bytes": kv_stride,
           "segments": 2, "size_bytes": size, "save_ids": save_ids, "load_ids": load_ids}
    for l in range(layers):
        buf = random_bytes(size, layer_seed(7, l))
        out[f"input_{l}"] = buf.copy()
        kept, kr, vr = brute_save(buf, nb, bpb, kv_stride, 2, save_ids.tolist())
        out[f"host_k_{l}"] = kr
        out[f"host_v_{l}"] = vr
        brute_load(buf, nb, bpb, kv_stride, 2, load_ids.tolist(), kr, vr)
        out[f"restored_{l}"] = buf
    np.savez(os.path.join(HERE, "tiny_kvfirst.npz"), **out)


def make_tiny_blocks():
    # [6 blocks, 4 tokens, 8] bf16: one segment of 64 B per block.
    nb, bpb, layers = 6, 4 * 8 * 2, 2
    size = nb * bpb
    save_ids = np.array([4, 0, -3, 5], np.int32)
    load_ids = np.array([2, 1, 3], np.int32)
    out = {"num_blocks": nb, "bytes_per_block": bpb, "kv_stride_bytes": 0,
           "segments": 1, "size_bytes": size, "save_ids": save_ids, "load_ids": load_ids}
    for l in range(layers):
        buf = random_bytes(size, layer_seed(11, l))
        out[f"input_{l}"] = buf.copy()
        kept, region, _ = brute_save(buf, nb, bpb, 0, 1, save_ids.tolist())
        out[f"host_{l}"] = region
        brute_load(buf, nb, bpb, 0, 1, load_ids.tolist(), region, None)
        out[f"restored_{l}"] = buf
    np.savez(os.path.join(HERE, "tiny_blocks.npz"), **out)


def make_gpt2():
    # Config 1: 12 layers of fp16 [2, 512, 16, 12, 64]; 64 random saved blocks,
    # loaded back into 64 other random blocks.
    layers, nb, bpb = 12, 512, 16 * 12 * 64 * 2
    kv_stride = nb * bpb
    size = 2 * kv_stride
    seed = 0
    rng = np.random.Generator(np.random.PCG64(seed))
    save_ids = rng.choice(nb, 64, replace=False)
    rest = np.setdiff1d(np.arange(nb), save_ids)
    load_ids = rng.choice(rest, 64, replace=False)
    rec = {"workload": "gpt2 fp16 [2,512,16,12,64] x 12 layers", "layers": layers,
           "num_blocks": nb, "bytes_per_block": bpb, "kv_stride_bytes": kv_stride,
           "segments": 2, "size_bytes": size, "base_seed": seed,
           "save_ids": save_ids.tolist(), "load_ids": load_ids.tolist(),
           "host_k_sha256": [], "host_v_sha256": [], "restored_sha256": []}
    for l in range(layers):
        buf = random_bytes(size, layer_seed(seed, l))
        _, kr, vr = brute_save(buf, nb, bpb, kv_stride, 2, save_ids.tolist())
        rec["host_k_sha256"].append(sha(kr))
        rec["host_v_sha256"].append(sha(vr))
        brute_load(buf, nb, bpb, kv_stride, 2, load_ids.tolist(), kr, vr)
        rec["restored_sha256"].append(sha(buf))
    with open(os.path.join(HERE, "gpt2_config1.json"), "w") as f:
        json.dump(rec, f, indent=1)


def make_packed():
    out = {}
    # Split: 2 layers x tp 2, slot = layer * 2 + rank; blocks in seal order.
    nb, bpb, layers, tp = 8, 32, 2, 2
    kv_stride, size = nb * bpb, 2 * nb * bpb
    ids = [5, 2, 7]
    slots = []
    for l in range(layers):
        for r in range(tp):
            buf = random_bytes(size, layer_seed(23 + r, l))
            out[f"split_input_{l}_{r}"] = buf
            slots.append(segment_view(buf, nb, bpb, kv_stride, 2))  # [K|V, block, bpb]
    arr = np.stack([np.stack([sv[:, b, :] for sv in slots]) for b in ids])  # [b, slot, 2, bpb]
    out["split_ids"] = np.array(ids, np.int32)
    out["split_file"] = arr.reshape(-1).copy()
    blk = 2 * bpb * len(slots)
    out["split_offsets"] = np.arange(len(ids), dtype=np.uint64) * blk
    out["split_meta"] = np.array([json.dumps(
        {"file": "00000000-0000-4000-8000-000000000001.bin", "offset": int(o),
         "slots": [{"is_split": True, "size": 2 * bpb} for _ in slots],
         "total_slots": len(slots)}, separators=(",", ":")) for o in out["split_offsets"]])
    # Contiguous: 1 layer, tp 1, blocks-first [6, 64 B].
    nb, bpb = 6, 64
    buf = random_bytes(nb * bpb, layer_seed(29, 0))
    out["contig_input"] = buf
    ids = [4, 0]
    out["contig_ids"] = np.array(ids, np.int32)
    out["contig_file"] = buf.reshape(nb, bpb)[ids].reshape(-1).copy()
    out["contig_offsets"] = np.arange(len(ids), dtype=np.uint64) * bpb
    out["contig_meta"] = np.array([json.dumps(
        {"file": "00000000-0000-4000-8000-000000000002.bin", "offset": int(o),
         "slots": [{"is_split": False, "size": bpb}], "total_slots": 1},
        separators=(",", ":")) for o in out["contig_offsets"]])
    np.savez(os.path.join(HERE, "packed_tiny.npz"), **out)


if __name__ == "__main__":
    make_tiny_kvfirst()
    make_tiny_blocks()
    make_gpt2()
    make_packed()
    print("wrote fixtures to", HERE)
