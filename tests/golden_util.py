"""Helpers that turn the JSON fixtures into numpy arrays (test-side only)."""
import numpy as np

NP = {"f32": np.float32, "u8": np.uint8, "i8": np.int8, "i32": np.int32, "i64": np.int64}


def tensor(t):
    """A fixture tensor dict -> numpy array (floats rebuilt bit-exactly from 'bits')."""
    if t["dtype"] == "f32":
        a = np.array(t["bits"], dtype=np.uint32).view(np.float32)
    else:
        a = np.array(t["values"], dtype=NP[t["dtype"]])
    return a.reshape(t["dims"])


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
