"""Client of the `pegaflow.Engine` gRPC service.

Mirrors the reference's PyO3 EngineRpcClient (python/src/lib.rs:262-525):
the same methods, argument order and return shapes — (ok, message) tuples,
and a dict for query — so a connector written against it runs unchanged.
"""

from __future__ import annotations

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
            body = proto.SaveLayer(block_ids=[int(i) for i in block_ids],
                                   block_hashes=[bytes(h) for h in block_hashes])
            hit = bodies[key] = (block_ids, block_hashes, body.SerializeToString())
        layer = proto.SaveLayer(layer_name=layer_name).SerializeToString() + hit[2]
        parts += [_SAVES_TAG, _varint(len(layer)), layer]
    return b"".join(parts)


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
        req = proto.LoadRequest(instance_id=instance_id, tp_rank=tp_rank, device_id=device_id,
                                load_state_shm=load_state_shm, layer_names=list(layer_names),
                                block_ids=list(block_ids),
                                block_hashes=[bytes(h) for h in block_hashes])
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
