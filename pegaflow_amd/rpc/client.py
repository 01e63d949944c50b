"""Client of the `pegaflow.Engine` gRPC service.

Mirrors the reference's PyO3 EngineRpcClient (python/src/lib.rs:262-525):
the same methods, argument order and return shapes — (ok, message) tuples,
and a dict for query — so a connector written against it runs unchanged.
"""

from __future__ import annotations

import operator

import grpc

from . import proto

_STATE_NAMES = {proto.PREFETCH_READY: "ready", proto.PREFETCH_LOADING: "loading",
                proto.PREFETCH_PARTIAL_MISS: "partial_miss"}


def _varint(n: int) -> bytes:
    out = bytearray()
    while True:
        b, n = n & 0x7F, n >> 7
        if not n:
            out.append(b)
            return bytes(out)
        out.append(b | 0x80)


_SAVES_TAG = _varint((proto.SaveRequest.DESCRIPTOR.fields_by_name["saves"].number << 3) | 2)


def _ids_part(msg_cls, block_ids) -> bytes:
    """The packed int32 block_ids field of `msg_cls` alone.  The message
    takes ints and numpy integers as they are; other integer-like values
    (bools) are converted first, and non-integers raise TypeError."""
    if not isinstance(block_ids, (list, tuple)) and not hasattr(block_ids, "__array__"):
        block_ids = list(block_ids)  # an iterator is read once
    try:
        return msg_cls(block_ids=block_ids).SerializeToString()
    except TypeError:
        return msg_cls(block_ids=[operator.index(i) for i in block_ids]).SerializeToString()


def _hashes_part(msg_cls, block_hashes) -> bytes:
    """The repeated bytes block_hashes field of `msg_cls` alone.  Hashes of
    one length under 128 bytes (a one-byte length) share the two-byte
    tag + length prefix, so the field is one join of the hashes; any other
    list is serialized by the message."""
    if not isinstance(block_hashes, (list, tuple)):
        block_hashes = list(block_hashes)
    if not block_hashes:
        return b""
    try:
        size = len(block_hashes[0])
        if size < 128 and set(map(len, block_hashes)) == {size}:
            field = msg_cls.DESCRIPTOR.fields_by_name["block_hashes"].number
            prefix = bytes(((field << 3) | 2, size))
            return prefix + prefix.join(block_hashes)
    except TypeError:
        pass
    return msg_cls(block_hashes=[bytes(h) for h in block_hashes]).SerializeToString()


def encode_save_request(instance_id: str, tp_rank: int, device_id: int, saves) -> bytes:
    """SaveRequest wire bytes for [(layer_name, block_ids, block_hashes)].

    The layers of a save usually share one id list and one hash list.  Each
    distinct pair is serialized once and every layer's SaveLayer is its name
    field followed by those bytes (two serialized parts of one message
    concatenate into the message with both), so the request costs one
    encoding of the lists instead of one per layer.  The cache holds each
    list it keys, so an id() cannot be reused within the call."""
    parts = [proto.SaveRequest(instance_id=instance_id, tp_rank=tp_rank,
                               device_id=device_id).SerializeToString()]
    bodies = {}
    for layer_name, block_ids, block_hashes in saves:
        key = (id(block_ids), id(block_hashes))
        hit = bodies.get(key)
        if hit is None or hit[0] is not block_ids or hit[1] is not block_hashes:
            body = (_ids_part(proto.SaveLayer, block_ids) +
                    _hashes_part(proto.SaveLayer, block_hashes))
            hit = bodies[key] = (block_ids, block_hashes, body)
        name = _NAME_FIELDS.get(layer_name)
        if name is None:  # a connector names the same layers every step
            if len(_NAME_FIELDS) >= 4096:
                _NAME_FIELDS.clear()
            name = _NAME_FIELDS[layer_name] = proto.SaveLayer(
                layer_name=layer_name).SerializeToString()
        parts += [_SAVES_TAG, _varint(len(name) + len(hit[2])), name, hit[2]]
    return b"".join(parts)


_NAME_FIELDS: dict = {}  # layer name -> its SaveLayer name field, serialized


_LAYER_NAMES_CACHE: dict = {}


def encode_load_request(instance_id: str, tp_rank: int, device_id: int, load_state_shm: str,
                        layer_names, block_ids, block_hashes) -> bytes:
    """LoadRequest wire bytes.  A connector names the same layers on every
    load, so the layer-name field is serialized once per name list (cached)
    and concatenated with the rest (serialized parts of one message
    concatenate into the message with all the fields)."""
    names = tuple(layer_names)
    named = _LAYER_NAMES_CACHE.get(names)
    if named is None:
        if len(_LAYER_NAMES_CACHE) >= 64:
            _LAYER_NAMES_CACHE.clear()
        named = _LAYER_NAMES_CACHE[names] = proto.LoadRequest(
            layer_names=list(names)).SerializeToString()
    head = proto.LoadRequest(instance_id=instance_id, tp_rank=tp_rank, device_id=device_id,
                             load_state_shm=load_state_shm).SerializeToString()
    return (head + named + _ids_part(proto.LoadRequest, block_ids) +
            _hashes_part(proto.LoadRequest, block_hashes))


def _serialize(request) -> bytes:
    """Requests are messages, or wire bytes already encoded."""
    return request if isinstance(request, bytes) else request.SerializeToString()


def _target(endpoint: str) -> str:
    for scheme in ("http://", "https://"):
        if endpoint.startswith(scheme):
            return endpoint[len(scheme):].rstrip("/")
    return endpoint


class EngineRpcClient:
    """python/src/lib.rs:262-291: connects eagerly and fails when the server
    does not answer within `connect_timeout_s`.  `endpoint` is
    "http://host:port" or "host:port"."""

    def __init__(self, endpoint: str | None = None, timeout_s: float | None = None,
                 connect_timeout_s: float = 2.0):
        self._endpoint = endpoint or "http://127.0.0.1:50055"
        self.timeout_s = timeout_s
        self._channel = grpc.insecure_channel(
            _target(self._endpoint),
            options=[("grpc.max_receive_message_length", 256 << 20),
                     ("grpc.max_send_message_length", 256 << 20),
                     ("grpc.keepalive_time_ms", 30000)])
        try:
            grpc.channel_ready_future(self._channel).result(timeout=connect_timeout_s)
        except grpc.FutureTimeoutError:
            self._channel.close()
            raise RuntimeError(f"failed to connect to engine server at {self._endpoint}: "
                               f"no answer within {connect_timeout_s} s") from None
        self._stubs = {
            rpc: self._channel.unary_unary(proto.method_path(rpc),
                                           request_serializer=_serialize,
                                           response_deserializer=proto.messages[resp].FromString)
            for rpc, req, resp in proto.METHODS}

    def close(self) -> None:
        self._channel.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _call(self, rpc: str, method: str, request):
        try:
            return self._stubs[rpc](request, timeout=self.timeout_s)
        except grpc.RpcError as err:
            code = err.code() if hasattr(err, "code") else None
            detail = err.details() if hasattr(err, "details") else str(err)
            raise RuntimeError(f"{method} RPC failed: status: {code}, message: {detail!r}") from None

    @staticmethod
    def _status(method: str, resp):
        if not resp.HasField("status"):
            raise RuntimeError(f"{method} response missing status")
        return resp.status.ok, resp.status.message

    def endpoint(self) -> str:
        return self._endpoint

    def health(self):
        return self._status("health", self._call("Health", "health", proto.HealthRequest()))

    def register_context(self, instance_id: str, namespace: str, tp_rank: int, tp_size: int,
                         device_id: int, num_layers: int, layer_name: str, wrapper_bytes: bytes,
                         num_blocks: int, bytes_per_block: int, kv_stride_bytes: int,
                         segments: int):
        """python/src/lib.rs:326-365 (argument order kept)."""
        req = proto.RegisterContextRequest(
            instance_id=instance_id, namespace=namespace, tp_rank=tp_rank, tp_size=tp_size,
            device_id=device_id, num_layers=num_layers, layer_name=layer_name,
            wrapper_bytes=bytes(wrapper_bytes), num_blocks=num_blocks,
            bytes_per_block=bytes_per_block, kv_stride_bytes=kv_stride_bytes, segments=segments)
        return self._status("register_context",
                            self._call("RegisterContext", "register_context", req))

    def save(self, instance_id: str, tp_rank: int, device_id: int, saves):
        """python/src/lib.rs:374-405: `saves` is [(layer_name, block_ids, block_hashes)]."""
        req = encode_save_request(instance_id, tp_rank, device_id, saves)
        return self._status("save", self._call("Save", "save", req))

    def load(self, instance_id: str, tp_rank: int, device_id: int, load_state_shm: str,
             layer_names, block_ids, block_hashes):
        """python/src/lib.rs:417-446."""
        req = encode_load_request(instance_id, tp_rank, device_id, load_state_shm, layer_names,
                                  block_ids, block_hashes)
        return self._status("load", self._call("Load", "load", req))

    def query(self, instance_id: str, block_hashes):
        """python/src/lib.rs:458-500: returns {ok, message, hit_blocks,
        prefetch_state, loading_blocks, missing_blocks}; an unknown state reads
        as "ready"."""
        resp = self._call("Query", "query", proto.QueryRequest(
            instance_id=instance_id, block_hashes=[bytes(h) for h in block_hashes]))
        ok, message = self._status("query", resp)
        return {"ok": ok, "message": message, "hit_blocks": resp.hit_blocks,
                "prefetch_state": _STATE_NAMES.get(resp.prefetch_state, "ready"),
                "loading_blocks": resp.loading_blocks, "missing_blocks": resp.missing_blocks}

    def unregister_context(self, instance_id: str):
        return self._status("unregister_context",
                            self._call("UnregisterContext", "unregister_context",
                                       proto.UnregisterRequest(instance_id=instance_id)))

    def shutdown(self):
        return self._status("shutdown", self._call("Shutdown", "shutdown",
                                                   proto.ShutdownRequest()))
