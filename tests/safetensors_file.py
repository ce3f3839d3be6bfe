"""Writes safetensors files for the weight-store tests: the format the
reference reads (u64 little-endian header length, JSON header, raw bytes)."""
import json
import struct

import numpy as np


def write(path, tensors, metadata=None, pad=True, header_override=None):
    """tensors: {name: (dtype_str, ndarray)}; BF16/F16 arrays are uint16 bit
    patterns.  Returns the header dict."""
    header, blobs, off = {}, [], 0
    for name, (dt, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    if metadata is not None:
        header["__metadata__"] = metadata
    text = (header_override if header_override is not None else json.dumps(header)).encode()
    if pad:
        text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)
    return header
