from .hip_runtime import HIPRuntime, HIPRuntimeError, HIPSafetyError, MemoryGuardianOOMError  # noqa: F401
from .memory import DeviceArray, MemoryRegion, SlabAllocator  # noqa: F401
