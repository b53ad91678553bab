"""Small helpers for GPU tests: upload numpy arrays, read them back."""
import numpy as np

from vte_amd.bridge import DeviceArray


def up(hip, arr, tag="t"):
    return DeviceArray.from_numpy(hip, np.ascontiguousarray(arr), tag)


def empty(hip, shape, dtype, tag="t"):
    d = DeviceArray(hip, shape, dtype, tag)
    d.zero()
    return d


def down(d):
    d.hip.synchronize()
    return d.numpy()
