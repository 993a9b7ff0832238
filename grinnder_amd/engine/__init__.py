"""Training engine: layer-wise, partition-wise orchestration."""


def __getattr__(name):
    if name == "Trainer":
        from grinnder_amd.engine.trainer import Trainer
        return Trainer
    if name == "StreamManager":
        from grinnder_amd.engine.streams import StreamManager
        return StreamManager
    raise AttributeError(f"module 'grinnder_amd.engine' has no attribute {name!r}")


__all__ = ["Trainer", "StreamManager"]
