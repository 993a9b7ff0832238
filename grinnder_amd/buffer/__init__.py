"""Host and device partition buffers."""

from grinnder_amd.buffer.device import DeviceBuffer
from grinnder_amd.buffer.host import HostBuffer

__all__ = ["HostBuffer", "DeviceBuffer"]
