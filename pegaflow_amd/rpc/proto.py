"""The `pegaflow.Engine` gRPC schema, built at run time.

Message and field names, numbers and types follow the reference's
pegaflow-proto/proto/engine.proto:5-115 exactly, so this server and client are
wire-compatible with the reference's tonic server and Rust/PyO3 client.  The
image has no protoc, so the descriptors are assembled with descriptor_pb2
instead of being generated.
"""

from __future__ import annotations

from typing import NamedTuple

from google.protobuf import descriptor_pb2, descriptor_pool, message_factory

PACKAGE = "pegaflow"
SERVICE = "Engine"

_F = descriptor_pb2.FieldDescriptorProto
_T = {
    "bool": _F.TYPE_BOOL,
    "string": _F.TYPE_STRING,
    "bytes": _F.TYPE_BYTES,
    "int32": _F.TYPE_INT32,
    "uint32": _F.TYPE_UINT32,
    "uint64": _F.TYPE_UINT64,
}

# (message, [(field, number, type, repeated)]) — engine.proto:5-105.
MESSAGES = [
    ("ResponseStatus", [("ok", 1, "bool", False), ("message", 2, "string", False)]),
    ("RegisterContextRequest", [
        ("instance_id", 1, "string", False), ("device_id", 2, "int32", False),
        ("layer_name", 3, "string", False), ("wrapper_bytes", 4, "bytes", False),
        ("num_blocks", 5, "uint64", False), ("bytes_per_block", 6, "uint64", False),
        ("kv_stride_bytes", 7, "uint64", False), ("segments", 8, "uint32", False),
        ("tp_rank", 9, "uint32", False), ("tp_size", 10, "uint32", False),
        ("num_layers", 11, "uint32", False), ("namespace", 12, "string", False)]),
    ("RegisterContextResponse", [("status", 1, ".pegaflow.ResponseStatus", False)]),
    ("SaveLayer", [("layer_name", 1, "string", False), ("block_ids", 2, "int32", True),
                   ("block_hashes", 3, "bytes", True)]),
    ("SaveRequest", [("instance_id", 1, "string", False), ("tp_rank", 2, "uint32", False),
                     ("device_id", 3, "int32", False),
                     ("saves", 4, ".pegaflow.SaveLayer", True)]),
    ("SaveResponse", [("status", 1, ".pegaflow.ResponseStatus", False)]),
    ("LoadRequest", [("instance_id", 1, "string", False), ("tp_rank", 2, "uint32", False),
                     ("device_id", 3, "int32", False), ("load_state_shm", 4, "string", False),
                     ("layer_names", 5, "string", True), ("block_ids", 6, "int32", True),
                     ("block_hashes", 7, "bytes", True)]),
    ("LoadResponse", [("status", 1, ".pegaflow.ResponseStatus", False)]),
    ("QueryRequest", [("instance_id", 1, "string", False), ("block_hashes", 2, "bytes", True)]),
    ("QueryResponse", [("status", 1, ".pegaflow.ResponseStatus", False),
                       ("hit_blocks", 2, "uint64", False),
                       ("prefetch_state", 3, "enum:.pegaflow.PrefetchState", False),
                       ("loading_blocks", 4, "uint64", False),
                       ("missing_blocks", 5, "uint64", False)]),
    ("UnregisterRequest", [("instance_id", 1, "string", False)]),
    ("UnregisterResponse", [("status", 1, ".pegaflow.ResponseStatus", False)]),
    ("ShutdownRequest", []),
    ("ShutdownResponse", [("status", 1, ".pegaflow.ResponseStatus", False)]),
    ("HealthRequest", []),
    ("HealthResponse", [("status", 1, ".pegaflow.ResponseStatus", False)]),
]

# engine.proto:66-74.
PREFETCH_READY, PREFETCH_LOADING, PREFETCH_PARTIAL_MISS = 0, 1, 2

# engine.proto:107-115: (rpc, request, response).
METHODS = [
    ("RegisterContext", "RegisterContextRequest", "RegisterContextResponse"),
    ("Save", "SaveRequest", "SaveResponse"),
    ("Load", "LoadRequest", "LoadResponse"),
    ("Query", "QueryRequest", "QueryResponse"),
    ("UnregisterContext", "UnregisterRequest", "UnregisterResponse"),
    ("Shutdown", "ShutdownRequest", "ShutdownResponse"),
    ("Health", "HealthRequest", "HealthResponse"),
]


def _file_proto() -> descriptor_pb2.FileDescriptorProto:
    fp = descriptor_pb2.FileDescriptorProto(name="pegaflow/engine.proto", package=PACKAGE,
                                            syntax="proto3")
    enum = fp.enum_type.add(name="PrefetchState")
    for name, num in (("PREFETCH_READY", 0), ("PREFETCH_LOADING", 1),
                      ("PREFETCH_PARTIAL_MISS", 2)):
        enum.value.add(name=name, number=num)
    for msg_name, fields in MESSAGES:
        m = fp.message_type.add(name=msg_name)
        for name, number, ftype, repeated in fields:
            f = m.field.add(name=name, number=number, json_name=_json_name(name))
            f.label = _F.LABEL_REPEATED if repeated else _F.LABEL_OPTIONAL
            if ftype.startswith("enum:"):
                f.type = _F.TYPE_ENUM
                f.type_name = ftype[5:]
            elif ftype.startswith("."):
                f.type = _F.TYPE_MESSAGE
                f.type_name = ftype
            else:
                f.type = _T[ftype]
    svc = fp.service.add(name=SERVICE)
    for rpc, req, resp in METHODS:
        svc.method.add(name=rpc, input_type=f".{PACKAGE}.{req}", output_type=f".{PACKAGE}.{resp}")
    return fp


def _json_name(name: str) -> str:
    head, *rest = name.split("_")
    return head + "".join(p.capitalize() for p in rest)


_pool = descriptor_pool.DescriptorPool()
FILE = _pool.Add(_file_proto())
_fd = _pool.FindFileByName("pegaflow/engine.proto")

messages = {name: message_factory.GetMessageClass(_fd.message_types_by_name[name])
            for name, _ in MESSAGES}
globals().update(messages)


def method_path(rpc: str) -> str:
    return f"/{PACKAGE}.{SERVICE}/{rpc}"


# ---- SaveRequest as the engine takes it ------------------------------------
# A save carries every layer's copy of the same ids and hashes.  A decoded
# request handed to the service object keeps equal neighbouring lists as one
# shared list object, which the engine packs and looks up once.


class DecodedSave(NamedTuple):
    instance_id: str
    tp_rank: int
    device_id: int
    saves: list  # [(layer_name, block_ids, block_hashes)], equal neighbours shared


def decoded_save(msg) -> DecodedSave:
    """A parsed SaveRequest as a DecodedSave (equal neighbours shared)."""
    saves, prev = [], None
    for s in msg.saves:
        ids, hashes = list(s.block_ids), list(s.block_hashes)
        if prev is not None and ids == prev[0] and hashes == prev[1]:
            ids, hashes = prev
        prev = (ids, hashes)
        saves.append((s.layer_name, ids, hashes))
    return DecodedSave(msg.instance_id, msg.tp_rank, msg.device_id, saves)
