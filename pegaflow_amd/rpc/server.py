"""The engine server: `pegaflow.Engine` over gRPC in front of PegaEngine.

Mirrors pegaflow-server/src/service.rs:19-405 (RPC semantics and the mapping
of engine errors to gRPC codes, service.rs:77-88); the request logic and the
tensor registry (registry.rs:41-176) live in ``pegaflow_amd.frontend``; and
the subset of the CLI (lib.rs:38-113) that concerns this path; the disk
tier's --dfs-root / --dfs-quota (lib.rs:98-112) turn it on directly, since
its index needs no Redis.

Run: python -m pegaflow_amd.rpc.server --addr 127.0.0.1:50055 --device 0 --pool-size 30gb
"""

from __future__ import annotations

import argparse
import ctypes
import logging
import signal
import sys
import threading
from concurrent import futures

import grpc
from google.protobuf.message import DecodeError

from .. import _lib
from ..engine import PegaEngine
from ..frontend import EngineFrontend, RegisterTensorError, TensorRegistry  # noqa: F401
from . import proto

log = logging.getLogger("pegaflow.server")

# service.rs:77-88.
_CODE = {
    _lib.PF_ERR_INVALID_ARGUMENT: grpc.StatusCode.INVALID_ARGUMENT,
    _lib.PF_ERR_INSTANCE_MISSING: grpc.StatusCode.FAILED_PRECONDITION,
    _lib.PF_ERR_WORKER_MISSING: grpc.StatusCode.FAILED_PRECONDITION,
    _lib.PF_ERR_TOPOLOGY_MISMATCH: grpc.StatusCode.FAILED_PRECONDITION,
}


def parse_memory_size(s: str) -> int:
    """utils.rs:3-36: a number with an optional kb/mb/gb/tb suffix (1024-based)."""
    s = s.strip()
    if "_" in s:
        raise ValueError(f"Invalid number: '{s}'")
    boundary = next((i for i, c in enumerate(s) if c.isascii() and c.isalpha()), len(s))
    num, unit = s[:boundary].strip(), s[boundary:].strip().lower()
    try:
        value = float(num)
    except ValueError:
        raise ValueError(f"Invalid number: '{num}'") from None
    if value < 0:
        raise ValueError("Memory size cannot be negative")
    mult = {"": 1, "b": 1, "kb": 1 << 10, "mb": 1 << 20, "gb": 1 << 30, "tb": 1 << 40}
    if unit not in mult:
        raise ValueError(f"Unknown unit: '{unit}'. Use kb, mb, gb, or tb")
    return int(value * mult[unit])


def _ok():
    return proto.ResponseStatus(ok=True, message="")


class EngineService:
    """service.rs:133-405: the gRPC face of an ``EngineFrontend``."""

    def __init__(self, engine: PegaEngine, disk: bool = False):
        self.frontend = EngineFrontend(engine, disk=disk)
        self.engine = engine
        self.registry = self.frontend.registry
        self.shutdown_event = threading.Event()

    @staticmethod
    def _abort(context, err: Exception):
        if isinstance(err, RegisterTensorError):  # map_py_error, service.rs:90-93
            context.abort(grpc.StatusCode.INTERNAL, str(err))
        if isinstance(err, _lib.PegaFlowError):
            context.abort(_CODE.get(err.code, grpc.StatusCode.INTERNAL), str(err))
        context.abort(grpc.StatusCode.INTERNAL, str(err))

    def RegisterContext(self, req, context):
        try:
            self.frontend.register_context(req.instance_id, req.namespace, req.tp_rank,
                                           req.tp_size, req.device_id, req.num_layers,
                                           req.layer_name, req.wrapper_bytes, req.num_blocks,
                                           req.bytes_per_block, req.kv_stride_bytes, req.segments)
        except Exception as e:
            self._abort(context, e)
        return proto.RegisterContextResponse(status=_ok())

    # Save and Load arrive as their wire bytes (registered without a
    # deserializer) and are decoded by the engine itself, as on its native
    # endpoint.  A decoded message (a caller of the service object) takes the
    # Python path: layers that carry the same ids and hashes share one list
    # object, which the engine packs and looks up once.
    def Save(self, req, context):
        try:
            if isinstance(req, bytes):
                self.frontend.serve(_lib.REQUEST_SAVE, req)
            else:
                if not isinstance(req, proto.DecodedSave):
                    req = proto.decoded_save(req)
                self.frontend.save(req.instance_id, req.tp_rank, req.device_id, req.saves)
        except Exception as e:
            self._abort(context, e)
        return proto.SaveResponse(status=_ok())

    def Load(self, req, context):
        try:
            if isinstance(req, bytes):
                self.frontend.serve(_lib.REQUEST_LOAD, req)
            else:
                self.frontend.load(req.instance_id, req.tp_rank, req.device_id,
                                   req.load_state_shm, req.layer_names, req.block_ids,
                                   req.block_hashes)
        except Exception as e:
            self._abort(context, e)
        return proto.LoadResponse(status=_ok())

    def Query(self, req, context):
        """service.rs:258-330: with a disk tier, a miss that is on disk starts
        a read into the pinned pool and is reported as loading."""
        try:
            q = self.frontend.query(req.instance_id, req.block_hashes)
        except Exception as e:
            self._abort(context, e)
        return proto.QueryResponse(status=_ok(), hit_blocks=q["hit_blocks"],
                                   prefetch_state=q["state"], loading_blocks=q["loading_blocks"],
                                   missing_blocks=q["missing_blocks"])

    def UnregisterContext(self, req, context):
        try:
            self.frontend.unregister(req.instance_id)
        except Exception as e:
            self._abort(context, e)
        return proto.UnregisterResponse(status=_ok())

    def Shutdown(self, req, context):
        log.warning("Shutdown requested via RPC")
        self.shutdown_event.set()
        return proto.ShutdownResponse(status=_ok())

    def Health(self, req, context):
        return proto.HealthResponse(status=_ok())

    def handler(self) -> grpc.GenericRpcHandler:
        methods = {}
        for rpc, req, resp in proto.METHODS:
            methods[rpc] = grpc.unary_unary_rpc_method_handler(
                getattr(self, rpc),
                request_deserializer=(None if rpc in ("Save", "Load")
                                      else proto.messages[req].FromString),
                response_serializer=proto.messages[resp].SerializeToString)
        return grpc.method_handlers_generic_handler(f"{proto.PACKAGE}.{proto.SERVICE}", methods)


class _Abort(Exception):
    def __init__(self, code: grpc.StatusCode, details: str):
        super().__init__(details)
        self.code, self.details = code, details


class _CallContext:
    """What the service's handlers use of a grpc.ServicerContext."""

    def abort(self, code, details):
        raise _Abort(code, details)


class NativeGrpc:
    """The Engine service on the library's native gRPC server
    (pf_grpc_start): Load, Save and Health are served by the engine on the
    server's own threads; the other RPCs reach ``service`` through a
    callback, with the same results, codes and messages as on grpcio."""

    def __init__(self, engine: PegaEngine, service: EngineService, addr: str):
        self._methods = {rpc: (getattr(service, rpc), proto.messages[req])
                         for rpc, req, _ in proto.METHODS}
        self._lib = _lib.load()
        self._cb = _lib.GRPC_HANDLER(self._handle)  # kept alive with the server
        h = ctypes.c_void_p()
        rc = self._lib.pf_grpc_start(engine._h, addr.encode(), self._cb, None, ctypes.byref(h))
        if rc != _lib.PF_OK:
            raise RuntimeError(f"failed to bind {addr}: {_lib.last_error()}")
        self._h = h.value
        self.port = int(self._lib.pf_grpc_port(self._h))

    def _handle(self, _ctx, call, method, request, size):
        # Nothing may escape a ctypes callback: every outcome is a reply.
        out, status, msg = b"", 0, None
        try:
            fn, req_cls = self._methods[method.decode()]
            req = req_cls.FromString(ctypes.string_at(request, size) if size else b"")
            out = fn(req, _CallContext()).SerializeToString()
        except KeyError:
            status, msg = grpc.StatusCode.UNIMPLEMENTED.value[0], "Method not found!"
        except DecodeError:
            status, msg = grpc.StatusCode.INTERNAL.value[0], "Exception deserializing request!"
        except _Abort as a:
            status, msg = a.code.value[0], a.details
        except Exception as e:  # noqa: BLE001 - reported to the caller as INTERNAL
            status, msg = grpc.StatusCode.INTERNAL.value[0], str(e) or type(e).__name__
        self._lib.pf_grpc_reply(call, status, msg.encode() if msg else None, out, len(out))

    def served(self) -> int:
        return int(self._lib.pf_grpc_served(self._h)) if self._h else 0

    def stop(self) -> None:
        if self._h:
            self._lib.pf_grpc_stop(self._h)
        self._h = None


class Server:
    """A running engine server (engine + registry + gRPC endpoint).

    grpc_impl "native" (the default) serves gRPC from the library's own
    HTTP/2 server (NativeGrpc); "python" from grpcio's server."""

    def __init__(self, addr: str = "127.0.0.1:50055", engine: PegaEngine | None = None,
                 pool_size: int = 30 << 30, host_pool: bool = False, unit_size_hint: int = 0,
                 max_workers: int = 16, dfs_root: str | None = None,
                 dfs_quota: int = 50 << 30, dfs_io_threads: int = 4,
                 grpc_impl: str = "native",
                 save_mode: int | None = None, load_mode: int | None = None,
                 lfu_admission: bool = False, pre_evict: bool = False,
                 pre_evict_threshold: int = 5 << 30, pre_evict_target: int = 8 << 30,
                 pre_evict_interval_ms: int = 100):
        self.engine = engine or PegaEngine(pool_size=pool_size, host_pool=host_pool,
                                           unit_size_hint=unit_size_hint)
        if lfu_admission or pre_evict:
            self.engine.set_storage_policy(lfu_admission, unit_size_hint, pre_evict,
                                           pre_evict_threshold, pre_evict_target,
                                           pre_evict_interval_ms)
        if dfs_root:
            self.engine.enable_disk(dfs_root, quota_bytes=dfs_quota, io_threads=dfs_io_threads)
        if save_mode is not None or load_mode is not None:
            self.engine.set_transfer_modes(_lib.MODE_AUTO if save_mode is None else save_mode,
                                           _lib.MODE_AUTO if load_mode is None else load_mode)
        self.service = EngineService(self.engine, disk=bool(dfs_root))
        self.grpc = self.native = None
        if grpc_impl == "native":
            self.native = NativeGrpc(self.engine, self.service, addr)
            self.port = self.native.port
        elif grpc_impl == "python":
            self.grpc = grpc.server(futures.ThreadPoolExecutor(max_workers=max_workers),
                                    options=[("grpc.max_receive_message_length", 256 << 20),
                                             ("grpc.max_send_message_length", 256 << 20)])
            self.grpc.add_generic_rpc_handlers((self.service.handler(),))
            self.port = self.grpc.add_insecure_port(addr)
            if self.port == 0:
                raise RuntimeError(f"failed to bind {addr}")
        else:
            raise ValueError(f"unknown gRPC implementation {grpc_impl!r}")
        self.grpc_impl = grpc_impl
        self.addr = addr.rsplit(":", 1)[0] + f":{self.port}"

    def start(self) -> "Server":
        if self.grpc is not None:
            self.grpc.start()
        log.info("pegaflow engine server listening on %s (%s gRPC)", self.addr, self.grpc_impl)
        return self

    def wait(self, poll_s: float = 0.2) -> None:
        while not self.service.shutdown_event.wait(poll_s):
            pass

    def stop(self, grace: float = 1.0) -> None:
        if self.native is not None:
            self.native.stop()
        if self.grpc is not None:
            self.grpc.stop(grace).wait()
        self.service.frontend.close()
        self.engine.close()


# The reference's default DFS root (pegaflow-server/src/lib.rs:98-104).
DEFAULT_DFS_ROOT = "/tmp/pega"


def parse_args(argv=None):
    """The reference's CLI (pegaflow-server/src/lib.rs:38-113), so its launch
    commands run unchanged, plus this server's own options.  Options for
    parts this server does not have are accepted and reported by
    unsupported_options()."""
    ap = argparse.ArgumentParser(prog="pegaflow-server",
                                 description="PegaEngine gRPC server (MI355X transfer path)")
    ap.add_argument("--addr", default="127.0.0.1:50055")
    ap.add_argument("--device", type=int, default=0)
    ap.add_argument("--pool-size", type=parse_memory_size, default=parse_memory_size("30gb"))
    ap.add_argument("--hint-value-size", type=parse_memory_size, default=0,
                    help="allocation unit of the pinned pool, and the value size TinyLFU "
                         "admission is sized for (128 MiB when not given)")
    ap.add_argument("--log-level", default="info")
    ap.add_argument("--max-workers", type=int, default=16,
                    help="worker threads of the python gRPC server")
    ap.add_argument("--save-mode", choices=sorted(_lib.MODE_NAMES), default="auto",
                    help="transfer mode of saves (auto: staged on the copy engines for long "
                         "host runs)")
    ap.add_argument("--load-mode", choices=sorted(_lib.MODE_NAMES), default="auto",
                    help="transfer mode of loads (auto: staged for long host runs; kernel: "
                         "the zero-copy kernel throughout)")
    ap.add_argument("--grpc-impl", choices=("native", "python"), default="native",
                    help="serve gRPC from the library's native HTTP/2 server (default) or "
                         "from grpcio's")
    ap.add_argument("--dfs-root", default=None,
                    help="directory of the disk tier (packed block files); the tier is on when "
                         f"this or --redis-url is given (default root {DEFAULT_DFS_ROOT})")
    ap.add_argument("--dfs-quota", type=parse_memory_size, default=parse_memory_size("50gb"))
    ap.add_argument("--dfs-io-threads", type=int, default=4)
    ap.add_argument("--redis-url", default=None,
                    help="turns the disk tier on, as in the reference; its index is kept in "
                         "sidecar files next to the packed files, so Redis itself is not used")
    ap.add_argument("--dfs-scan-interval-ms", type=int, default=100,
                    help="accepted for compatibility (quota is enforced after every write)")
    ap.add_argument("--pre-evict", action="store_true",
                    help="evict least-recently-used blocks in the background while fewer than "
                         "--pre-evict-threshold bytes of the pool are free")
    ap.add_argument("--pre-evict-threshold", type=parse_memory_size,
                    default=parse_memory_size("5gb"))
    ap.add_argument("--pre-evict-target", type=parse_memory_size, default=parse_memory_size("8gb"))
    ap.add_argument("--pre-evict-interval-ms", type=int, default=100)
    ap.add_argument("--lfu-admission", action="store_true",
                    help="TinyLFU admission of new blocks, as the reference's server runs by "
                         "default (off here: sized for 128 MiB values, it refuses blocks by "
                         "sketch collisions; see --hint-value-size)")
    ap.add_argument("--disable-lfu-admission", action="store_true",
                    help="accepted for compatibility: admission is off unless --lfu-admission")
    # Reference options for parts this server does not have.
    ap.add_argument("--use-hugepages", action="store_true")
    ap.add_argument("--metrics-otel-endpoint", default="http://127.0.0.1:4321")
    ap.add_argument("--metrics-period-secs", type=int, default=5)
    args = ap.parse_args(argv)
    if args.dfs_root is None and args.redis_url:
        args.dfs_root = DEFAULT_DFS_ROOT
    return args


def unsupported_options(args) -> list[str]:
    """Reference options given on the command line that change nothing here."""
    out = []
    if args.use_hugepages:
        out.append("--use-hugepages: the pool is hipHostMalloc memory (registering existing "
                   "huge pages is refused on this platform)")
    return out


def main(argv=None) -> int:
    args = parse_args(argv)
    logging.basicConfig(level=getattr(logging, args.log_level.upper(), logging.INFO),
                        format="%(asctime)s %(levelname)s %(name)s: %(message)s")
    for msg in unsupported_options(args):
        log.warning("option without effect in this server: %s", msg)
    from .. import runtime
    runtime.init(args.device)
    server = Server(args.addr, pool_size=args.pool_size, unit_size_hint=args.hint_value_size,
                    max_workers=args.max_workers, dfs_root=args.dfs_root,
                    dfs_quota=args.dfs_quota, dfs_io_threads=args.dfs_io_threads,
                    grpc_impl=args.grpc_impl,
                    save_mode=_lib.MODE_NAMES[args.save_mode],
                    load_mode=_lib.MODE_NAMES[args.load_mode],
                    lfu_admission=args.lfu_admission and not args.disable_lfu_admission,
                    pre_evict=args.pre_evict, pre_evict_threshold=args.pre_evict_threshold,
                    pre_evict_target=args.pre_evict_target,
                    pre_evict_interval_ms=args.pre_evict_interval_ms).start()
    for sig in (signal.SIGINT, signal.SIGTERM):
        signal.signal(sig, lambda *_: server.service.shutdown_event.set())
    print(f"READY {server.addr}", flush=True)
    server.wait()
    server.stop()
    return 0


if __name__ == "__main__":
    sys.exit(main())
