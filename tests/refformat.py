"""Writes a model directory the way the reference's quantizer does (src/bin/quantize_model.rs:
284-306, manifest fields of src/storage/storage_manifest.rs:64-110): manifest.json with a
`layers` map, 4-bit projections as {id}_u4.bin + a separate `{id}.scale` layer in
{id}_scale.bin, int8 ones as {id}_i8.bin + {id}_scale.bin, everything else as {id}.bin f32
('.' in ids becomes '_'). Test infrastructure: the reference itself is never run."""
import hashlib
import json
import os

import numpy as np


def _meta(layer_id, shape, fmt, stored, bits=None, checksum=""):
    n = int(np.prod(shape))
    return {"layer_id": layer_id, "shape": list(shape), "num_elements": n, "original_bytes": n * 4,
            "stored_bytes": stored, "compression_format": fmt, "storage_tier": "Important",
            "reference_tensor": None, "statistics": {"access_count": 0, "last_accessed_timestamp": None},
            "quantization_bits": bits, "reference_layer": None, "checksum": checksum, "svd_rank": None}


def write_reference_dir(path, cfg, weights, checksums=True):
    """weights: (name, data, scales) as model.synth_weights / tinymodels.tiny_weights yield them,
    projections in BH_Q4_ROW (u8 + f32 scales) or BH_Q8_ROW (i8 + f32 scales)."""
    os.makedirs(path, exist_ok=True)
    layers = {}

    def put(fname, arr):
        arr = np.ascontiguousarray(arr)
        arr.tofile(os.path.join(path, fname))
        return hashlib.sha256(arr.tobytes()).hexdigest() if checksums else ""

    for name, data, scales in weights:
        safe = name.replace(".", "_")
        data = np.asarray(data)
        if scales is not None:
            n = data.shape[0]
            k = data.shape[1] * (2 if data.dtype == np.uint8 else 1)
            suffix, fmt, bits = ("_u4.bin", "Int4PerChannel", 4) if data.dtype == np.uint8 else ("_i8.bin", "Int8Linear", 8)
            ck = put(safe + suffix, data)
            layers[name] = _meta(name, (n, k), fmt, data.nbytes, bits, ck)
            ck = put(safe + "_scale.bin", np.asarray(scales, np.float32))
            layers[name + ".scale"] = _meta(name + ".scale", (n,), "None", n * 4, None, ck)
        else:
            arr = data.astype(np.float32)
            ck = put(safe + ".bin", arr)
            layers[name] = _meta(name, arr.shape, "None", arr.nbytes, None, ck)
    manifest = {"name": "tiny", "variant": "q4", "num_layers": cfg.n_layers, "architecture": "qwen2",
                "hidden_size": cfg.hidden, "num_heads": cfg.n_heads, "num_kv_heads": cfg.n_kv_heads,
                "layers": layers}
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2)
