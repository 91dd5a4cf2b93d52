"""Extract fp8-e4m3fn encoder byte pairs from the reference's committed fixtures.

The reference ships f32 models next to their fp8 repacks:

- ``tests/fixtures/tiny-mmdit/model.safetensors`` -> ``model_fp8.safetensors``
  (per-tensor 0-d scales),
- ``tests/fixtures/tiny-krea2/raw.safetensors`` -> ``turbo_fp8.safetensors``
  (one per-output-channel tensor, ``blocks.0.mlp.gate.weight`` [256, 64]).

Those pairs were written by ``reference/fp8_reference.py:83-91`` (scale =
amax/448, byte = RNE(w/scale)), so they pin an fp8 encoder byte-for-byte.
This script copies a bounded subset of them (inputs, expected bytes, expected
scales) into ``fp8_pairs.npz`` next to it. It parses the safetensors
container directly (8-byte little-endian header length, JSON header, raw
little-endian payload) and never imports or runs reference code.

Run in the build container only (``/root/reference`` does not exist on the GPU
box): ``python tests/golden/make_fp8_pairs.py``.
"""

import json
import os
import struct

import numpy as np

FIX = "/root/reference/crates/loractl-core/tests/fixtures"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fp8_pairs.npz")

_DT = {"F32": np.float32, "F8_E4M3": np.uint8, "BF16": np.uint16, "F16": np.float16}


def read_safetensors(path):
    """Return {name: (dtype_str, shape, ndarray)} without executing anything."""
    with open(path, "rb") as f:
        blob = f.read()
    (hlen,) = struct.unpack("<Q", blob[:8])
    header = json.loads(blob[8 : 8 + hlen])
    base = 8 + hlen
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        dt = meta["dtype"]
        if dt not in _DT:
            continue
        lo, hi = meta["data_offsets"]
        arr = np.frombuffer(blob[base + lo : base + hi], dtype=_DT[dt]).copy()
        out[name] = (dt, tuple(meta["shape"]), arr.reshape(meta["shape"]))
    return out


def pairs(src, dst, limit_elems):
    a = read_safetensors(os.path.join(FIX, src))
    b = read_safetensors(os.path.join(FIX, dst))
    picked = []
    total = 0
    for name in sorted(b):
        dt, shape, arr = b[name]
        if dt != "F8_E4M3" or len(shape) != 2:
            continue
        sdt, sshape, sarr = b[name + "_scale"]
        assert sdt == "F32"
        src_dt, src_shape, w = a[name]
        assert src_dt == "F32" and src_shape == shape, name
        per_channel = sarr.size > 1
        if total + w.size > limit_elems and not per_channel:
            continue
        picked.append((name, w.astype(np.float32), arr.astype(np.uint8), sarr.astype(np.float32).reshape(-1)))
        total += w.size
    return picked


def main():
    out = {}
    names = []
    for tag, (src, dst, lim) in {
        "mmdit": ("tiny-mmdit/model.safetensors", "tiny-mmdit/model_fp8.safetensors", 40000),
        "krea2": ("tiny-krea2/raw.safetensors", "tiny-krea2/turbo_fp8.safetensors", 20000),
    }.items():
        for i, (name, w, q, s) in enumerate(pairs(src, dst, lim)):
            key = f"{tag}_{i}"
            out[key + "_w"] = w
            out[key + "_bytes"] = q
            out[key + "_scale"] = s
            names.append(f"{key}={tag}:{name}")
    out["names"] = np.array(names)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(names)} tensors")
    for n in names:
        print(" ", n)


if __name__ == "__main__":
    main()
