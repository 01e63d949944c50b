"""Wire surface of the engine: the `pegaflow.Engine` gRPC service
(pegaflow-server/src/service.rs) and its client (EngineRpcClient,
python/src/lib.rs:263-528)."""
