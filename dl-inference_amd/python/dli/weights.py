"""dli.weights.v1 writer: the format include/dli/weights.h loads (reference writer:
python/dli_export/weights.py:18-62). One JSON manifest {format, data, tensors{name: {dtype,
shape, offset, nbytes}}} next to one binary blob; the names follow the reference's
<stem>.dli.weights.json / <stem>.dli.weights.bin. Besides the reference's float32 and int64,
bfloat16, float16 and int32 tensors are written as they are (no widening to float32), and every
tensor starts at a 64-byte aligned offset."""
from __future__ import annotations

import json
from pathlib import Path

import torch

_DTYPES = {torch.float32: "float32", torch.int64: "int64", torch.bfloat16: "bfloat16",
           torch.float16: "float16", torch.int32: "int32"}
_ALIGN = 64


def save_weights(output_dir, stem: str, tensors: dict) -> Path:
    """Writes tensors (name -> torch.Tensor, any device) and returns the manifest path."""
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    data_name = f"{stem}.dli.weights.bin"
    meta = {}
    offset = 0
    with (out / data_name).open("wb") as data:
        for name, tensor in tensors.items():
            host = tensor.detach().cpu().contiguous()
            if host.dtype not in _DTYPES:
                raise TypeError(f"unsupported tensor dtype for {name}: {host.dtype}")
            # raw bytes; 16-bit floats through an integer view (numpy has no bfloat16)
            raw = host.view(torch.int16) if host.element_size() == 2 else host
            payload = raw.numpy().tobytes()
            pad = (-offset) % _ALIGN
            data.write(b"\0" * pad)
            offset += pad
            meta[name] = {"dtype": _DTYPES[host.dtype], "shape": list(host.shape),
                          "offset": offset, "nbytes": len(payload)}
            data.write(payload)
            offset += len(payload)
    manifest = {"format": "dli.weights.v1", "data": data_name, "tensors": meta}
    path = out / f"{stem}.dli.weights.json"
    path.write_text(json.dumps(manifest, indent=2), encoding="utf-8")
    return path
