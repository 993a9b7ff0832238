"""Training engine: the layer-wise, partition-wise Trainer and its streams."""

from grinnder_amd.engine.streams import StreamManager
from grinnder_amd.engine.trainer import Trainer

__all__ = ["StreamManager", "Trainer"]
