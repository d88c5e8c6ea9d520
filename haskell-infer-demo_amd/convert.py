#!/usr/bin/env python3
"""Offline converter: BF16 dense-FFN weights -> INT4 artifacts + weights.manifest.json.

Writes the sidecar schema the reference converter writes and its reader enforces (reference
scripts/quantize_weights.py:42-64 format block, :219-318 entries / pairs / precision map /
manifest; csrc/quant_manifest.c), so a directory written here loads through
engine_load_quantized_ffn and through the reference's own reader alike. The arithmetic is the
library's quantizer (w4a16_quantize_int4, the format's rule from reference
csrc/linear_weight.cpp:108-176); this file is I/O and bookkeeping.

Layout on disk (as the reference's):
    OUT/weights.manifest.json
    OUT/artifacts/<role>_layer<L>.packed   u8 [N, K/2], lower K index in the low nibble
    OUT/artifacts/<role>_layer<L>.scales   bf16 [N, K/128]
    OUT/artifacts/mlpGateUp_layer<L>.*     the F1 pair: gate rows then up rows

Usage (BF16 safetensors checkpoint + the reference's descriptor JSON):
    python convert.py --model-dir DIR --desc descriptor.json --out-dir OUT
"""

import argparse
import hashlib
import json
import os
import struct
import sys

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

FORMAT = {
    "name": "int4_symmetric_group_bf16_scale",
    "abi_version": 1,
    "group": 128,
    "qmin": -7,
    "qmax": 7,
    "invalid_code": -8,
    "zero_point": 0,
    "packed_dtype": "u8",
    "scale_dtype": "bf16",
    "packing": "two_twos_complement_nibbles_per_byte_lower_k_index_in_low_nibble",
    "arithmetic": "w4a16_quantize_int4 (haskell-infer-demo_amd/csrc/format.cpp)",
}
MANIFEST_VERSION = 1
CONVERTER = {"name": "haskell-infer-demo_amd/convert.py", "version": 1}
ROLES = ("mlpGate", "mlpUp", "mlpDown")
PAIR_ROLES = ("mlpGate", "mlpUp")
PAIR_NAME = "mlpGateUp"


def _sha256(data):
    return hashlib.sha256(data).hexdigest()


def _artifact(out_dir, name, data, dtype, count=None):
    path = os.path.join(out_dir, "artifacts", name)
    with open(path, "wb") as handle:
        handle.write(data)
    art = {"file": f"artifacts/{name}", "dtype": dtype, "bytes": len(data), "sha256": _sha256(data)}
    if count is not None:
        art["count"] = count
    return art


def write_sidecar(out_dir, layers, model_dir, role_names=None, tensor_names=None, files=()):
    """Quantize and write every layer's FFN roles.

    layers: {layer: {"mlpGate": w, "mlpUp": w, "mlpDown": w}} with FP32 (BF16-valued) 2-D
    arrays; layers absent from the dict keep BF16. role_names: the descriptor's role list (for
    role_index and the precision map; defaults to the three FFN roles). tensor_names:
    {(layer, role): checkpoint tensor name}. Returns the manifest dict.
    """
    import w4a16

    role_names = list(role_names or ROLES)
    tensor_names = tensor_names or {}
    os.makedirs(os.path.join(out_dir, "artifacts"), exist_ok=True)
    entries, pairs, err_max, err_sq, err_n = [], [], 0.0, 0.0, 0
    raw = {}
    for layer in sorted(layers):
        for role in ROLES:
            if role not in layers[layer]:
                continue
            w = np.ascontiguousarray(layers[layer][role], dtype=np.float32)
            n, k = w.shape
            packed, scales = w4a16.quantize_int4(w)
            deq = w4a16.dequantize_int4(packed, scales, n, k)
            diff = np.abs(w.astype(np.float64) - deq)
            err_max = max(err_max, float(diff.max()))
            err_sq += float((diff ** 2).sum())
            err_n += diff.size
            pb, sb = packed.tobytes(), scales.tobytes()
            raw[(layer, role)] = (pb, sb, n, k)
            stem = f"{role}_layer{layer}"
            entries.append({
                "role": role,
                "role_index": role_names.index(role) if role in role_names else -1,
                "layer": layer,
                "checkpoint_tensor": tensor_names.get((layer, role), f"layer{layer}.{role}"),
                "logical_shape": [n, k],
                "local_shape": [n, k],
                "packed": _artifact(out_dir, f"{stem}.packed", pb, "u8"),
                "scales": _artifact(out_dir, f"{stem}.scales", sb, "bf16", len(sb) // 2),
                "group_axis": "k",
                "group": FORMAT["group"],
            })
    for layer in sorted(layers):
        if not all((layer, r) in raw for r in PAIR_ROLES):
            continue
        (gp, gs, gn, gk), (up, us, un, uk) = (raw[(layer, r)] for r in PAIR_ROLES)
        if gk != uk:
            raise ValueError(f"layer {layer}: gate and up differ in K")
        stem = f"{PAIR_NAME}_layer{layer}"
        pairs.append({
            "name": PAIR_NAME,
            "layer": layer,
            "members": [{"role": r, "role_index": role_names.index(r) if r in role_names else -1}
                        for r in PAIR_ROLES],
            "rule": "row concatenation: gate rows then up rows",
            "logical_shape": [gn + un, gk],
            "packed": _artifact(out_dir, f"{stem}.packed", gp + up, "u8"),
            "scales": _artifact(out_dir, f"{stem}.scales", gs + us, "bf16", (len(gs) + len(us)) // 2),
            "group": FORMAT["group"],
        })
    n_layers = (max(layers) + 1) if layers else 0
    precision_map = []
    for layer in range(n_layers):
        for role in role_names:
            precision_map.append({
                "role": role,
                "layer": layer,
                "precision": "int4" if (layer, role) in raw else "bf16",
                "checkpoint_tensor": tensor_names.get((layer, role), f"layer{layer}.{role}"),
            })
    manifest = {
        "manifest_version": MANIFEST_VERSION,
        "format": FORMAT,
        "converter": CONVERTER,
        "source": {"model_dir": os.path.abspath(model_dir), "files": list(files)},
        "quantization_error": {"max_abs": err_max, "rms": (err_sq / err_n) ** 0.5 if err_n else 0.0,
                               "elements": err_n,
                               "note": "against the FP32 source values, per element"},
        "precision_map": precision_map,
        "entries": entries,
        "pairs": pairs,
    }
    with open(os.path.join(out_dir, "weights.manifest.json"), "w") as handle:
        json.dump(manifest, handle, indent=2, sort_keys=True)
        handle.write("\n")
    return manifest


# ---- BF16 safetensors checkpoints ----------------------------------------------------------------

def read_safetensors_index(model_dir):
    """name -> (path, dtype, shape, start, stop) over every shard."""
    index = {}
    for name in sorted(os.listdir(model_dir)):
        if not name.endswith(".safetensors"):
            continue
        path = os.path.join(model_dir, name)
        with open(path, "rb") as handle:
            hlen = struct.unpack("<Q", handle.read(8))[0]
            header = json.loads(handle.read(hlen))
        for tensor, info in header.items():
            if tensor == "__metadata__":
                continue
            start, stop = info["data_offsets"]
            index[tensor] = (path, info["dtype"], list(info["shape"]), 8 + hlen + start, 8 + hlen + stop)
    return index


def read_bf16_as_f32(entry):
    path, dtype, shape, start, stop = entry
    if dtype != "BF16":
        raise ValueError(f"only BF16 sources are admitted, got {dtype}")
    with open(path, "rb") as handle:
        handle.seek(start)
        raw = handle.read(stop - start)
    return (np.frombuffer(raw, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(shape)


def convert_checkpoint(model_dir, desc_path, out_dir, limit_layers=None):
    with open(desc_path) as handle:
        desc = json.load(handle)
    names, templates = desc["role_names"], desc["role_templates"]
    index = read_safetensors_index(model_dir)
    layers, tensor_names = {}, {}
    for layer in range(desc["num_layers"]):
        if desc["layer_ffns"][layer] != "dense" or (limit_layers is not None and layer >= limit_layers):
            continue
        layers[layer] = {}
        for role in ROLES:
            template = templates[names.index(role)]
            tensor = template % layer if "%d" in template else template
            tensor_names[(layer, role)] = tensor
            layers[layer][role] = read_bf16_as_f32(index[tensor])
    files = []
    for name in sorted(os.listdir(model_dir)):
        if name.endswith(".safetensors"):
            with open(os.path.join(model_dir, name), "rb") as handle:
                data = handle.read()
            files.append({"name": name, "bytes": len(data), "sha256": _sha256(data)})
    return write_sidecar(out_dir, layers, model_dir, names, tensor_names, files)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--model-dir", required=True)
    ap.add_argument("--desc", required=True)
    ap.add_argument("--out-dir", required=True)
    ap.add_argument("--limit-layers", type=int)
    args = ap.parse_args()
    manifest = convert_checkpoint(args.model_dir, args.desc, args.out_dir, args.limit_layers)
    print(f"convert: {len(manifest['entries'])} entries, {len(manifest['pairs'])} pairs -> "
          f"{os.path.join(args.out_dir, 'weights.manifest.json')}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
