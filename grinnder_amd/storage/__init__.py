"""Storage tier: tensors spilled to files on local storage."""

from grinnder_amd.storage.backend import StorageBackend
from grinnder_amd.storage.tensor import StorageTensor

__all__ = ["StorageBackend", "StorageTensor"]
