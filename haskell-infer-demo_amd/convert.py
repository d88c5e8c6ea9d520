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
    python convert.py --verify OUT/weights.manifest.json [--reference QUANTIZER]

--verify re-derives the sidecar's claims the way the reference's --verify does (reference
scripts/quantize_weights.py:328-440): every artifact's size and digest, the source shards'
digests, the precision map covering every (layer, role) of the descriptor exactly once, each
pair being its members' rows in order, and a sample of entries re-quantized from the source
checkpoint (by this library, or by the reference's compiled quantizer when given).
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
    # The frozen format block is compared key by key by every reader, so it is the reference's
    # own text; "arithmetic" names the rule the artifacts follow (w4a16_quantize_int4
    # reproduces that quantizer bit for bit; tests/test_oracle.py pins it on golden vectors).
    "arithmetic": "csrc/linear_weight.cpp (the Q0 reference)",
}
MANIFEST_VERSION = 1
CONVERTER = {"name": "haskell-infer-demo_amd/convert.py", "version": 1}
ROLES = ("mlpGate", "mlpUp", "mlpDown")
PAIR_ROLES = ("mlpGate", "mlpUp")
PAIR_NAME = "mlpGateUp"


def _sha256(data):
    return hashlib.sha256(data).hexdigest()


def sha256_file(path, block=1 << 20):
    """Digest of a file read in 1 MiB blocks (a checkpoint shard is never held whole)."""
    digest = hashlib.sha256()
    with open(path, "rb") as handle:
        for chunk in iter(lambda: handle.read(block), b""):
            digest.update(chunk)
    return digest.hexdigest()


class ConvertError(ValueError):
    """A checkpoint, descriptor or sidecar the converter refuses."""


def _artifact(out_dir, name, data, dtype, count=None):
    path = os.path.join(out_dir, "artifacts", name)
    with open(path, "wb") as handle:
        handle.write(data)
    art = {"file": f"artifacts/{name}", "dtype": dtype, "bytes": len(data), "sha256": _sha256(data)}
    if count is not None:
        art["count"] = count
    return art


def write_sidecar(out_dir, layers, model_dir, role_names=None, tensor_names=None, files=(),
                  descriptor=None):
    """Quantize and write every layer's FFN roles.

    layers: {layer: {"mlpGate": w, "mlpUp": w, "mlpDown": w}} with FP32 (BF16-valued) 2-D
    arrays; layers absent from the dict keep BF16. role_names: the descriptor's role list (for
    role_index and the precision map; defaults to the three FFN roles). tensor_names:
    {(layer, role): checkpoint tensor name}. descriptor: {"path", "sha256"} of the descriptor
    the conversion followed (recorded as the reference converter does). Returns the manifest.
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
    if descriptor is not None and "num_layers" in descriptor:
        n_layers = max(n_layers, int(descriptor["num_layers"]))
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
        **({"descriptor": {"path": descriptor["path"], "sha256": descriptor["sha256"]}}
           if descriptor is not None else {}),
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
    """name -> (path, dtype, shape, start, stop) over every shard; a tensor named in two shards
    is refused (reference scripts/quantize_weights.py:72-92)."""
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
            if tensor in index:
                raise ConvertError(f"{tensor} appears in two shards")
            start, stop = info["data_offsets"]
            index[tensor] = (path, info["dtype"], list(info["shape"]), 8 + hlen + start, 8 + hlen + stop)
    return index


def read_bf16_as_f32(entry):
    """A BF16 tensor widened to FP32 (exact)."""
    path, dtype, shape, start, stop = entry
    if dtype != "BF16":
        raise ConvertError(f"only BF16 sources are admitted, got {dtype}")
    count = int(np.prod(shape)) if shape else 1
    if stop - start != 2 * count:
        raise ConvertError(f"{path}: a {shape} BF16 tensor spans {stop - start} bytes")
    with open(path, "rb") as handle:
        handle.seek(start)
        raw = handle.read(stop - start)
    return (np.frombuffer(raw, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(shape)


def _role_tensor(template, layer):
    return template % layer if "%d" in template else template


def _shard_records(model_dir):
    return [{"name": name, "bytes": os.path.getsize(os.path.join(model_dir, name)),
             "sha256": sha256_file(os.path.join(model_dir, name))}
            for name in sorted(os.listdir(model_dir)) if name.endswith(".safetensors")]


def convert_checkpoint(model_dir, desc_path, out_dir, limit_layers=None):
    """The reference converter's flow (scripts/quantize_weights.py:155-325) on this library's
    quantizer: the FFN roles of every dense layer of the descriptor, read from the BF16
    checkpoint, quantized, written with the F1 pair and the manifest. The source shards are
    hashed before and after, and a checkpoint that changed meanwhile is refused."""
    with open(desc_path) as handle:
        desc = json.load(handle)
    names, templates = desc["role_names"], desc["role_templates"]
    if len(names) != len(templates):
        raise ConvertError("the descriptor's role names and templates differ in length")
    for role in ROLES:
        if role not in names:
            raise ConvertError(f"the descriptor has no {role} role")
    before = _shard_records(model_dir)
    index = read_safetensors_index(model_dir)
    layers, tensor_names = {}, {}
    for layer in range(desc["num_layers"]):
        if desc["layer_ffns"][layer] != "dense" or (limit_layers is not None and layer >= limit_layers):
            continue
        layers[layer] = {}
        for role in ROLES:
            tensor = _role_tensor(templates[names.index(role)], layer)
            if tensor not in index:
                raise ConvertError(f"{tensor} is not in the checkpoint")
            w = read_bf16_as_f32(index[tensor])
            if w.ndim != 2:
                raise ConvertError(f"{tensor} is not a 2-D weight")
            tensor_names[(layer, role)] = tensor
            layers[layer][role] = w
    # every role of every layer in the precision map, named by its checkpoint tensor
    for layer in range(desc["num_layers"]):
        for role, template in zip(names, templates):
            tensor_names.setdefault((layer, role), _role_tensor(template, layer))
    if _shard_records(model_dir) != before:
        raise ConvertError("the source checkpoint changed during conversion")
    descriptor = {"path": os.path.abspath(desc_path), "sha256": sha256_file(desc_path),
                  "num_layers": desc["num_layers"]}
    return write_sidecar(out_dir, layers, model_dir, names, tensor_names, before, descriptor)


# ---- --verify -------------------------------------------------------------------------------

def _quantize_with(reference, w):
    """Payload and scales of w by the reference's compiled quantizer (its --quantize mode)."""
    import subprocess
    import tempfile

    n, k = w.shape
    with tempfile.TemporaryDirectory() as tmp:
        paths = [os.path.join(tmp, f) for f in ("in.f32", "out.packed", "out.scales")]
        with open(paths[0], "wb") as handle:
            handle.write(np.ascontiguousarray(w, dtype=np.float32).tobytes())
        proc = subprocess.run([reference, "--quantize", *paths, str(n), str(k)],
                              capture_output=True, text=True)
        if proc.returncode != 0:
            raise ConvertError(f"the reference quantizer refused [{n}, {k}]: {proc.stdout}{proc.stderr}")
        with open(paths[1], "rb") as handle:
            packed = handle.read()
        with open(paths[2], "rb") as handle:
            scales = handle.read()
    return packed, scales


def verify(manifest_path, reference=None, sample=2):
    """Re-derive a sidecar's claims; returns the list of problems (empty when it verifies)."""
    import w4a16

    with open(manifest_path) as handle:
        manifest = json.load(handle)
    out_dir = os.path.dirname(os.path.abspath(manifest_path))
    problems = []

    def require(ok, message):
        if not ok:
            problems.append(message)

    require(manifest.get("manifest_version") == MANIFEST_VERSION,
            f"unknown manifest version {manifest.get('manifest_version')}")
    for key, value in FORMAT.items():
        have = manifest.get("format", {}).get(key)
        require(have == value, f"the format's {key} is {have!r}, expected {value!r}")
    source_dir = manifest["source"]["model_dir"]
    for record in manifest["source"]["files"]:
        path = os.path.join(source_dir, record["name"])
        require(os.path.exists(path) and sha256_file(path) == record["sha256"],
                f"the source shard {record['name']} is missing or no longer matches its digest")

    def check_artifact(art, want_bytes, what):
        path = os.path.join(out_dir, art["file"])
        if not os.path.exists(path):
            problems.append(f"{what} has no artifact at {art['file']}")
            return False
        require(os.path.getsize(path) == want_bytes == art["bytes"],
                f"{what} is {os.path.getsize(path)} bytes, the shape needs {want_bytes}")
        require(sha256_file(path) == art["sha256"], f"{what} does not match its digest")
        return True

    seen, entries = {}, manifest["entries"]
    for e in entries:
        key = (e["layer"], e["role"])
        require(key not in seen, f"{key} appears twice")
        seen[key] = e
        n, k = e["logical_shape"]
        require(n % 8 == 0 and k % FORMAT["group"] == 0, f"{key} has a shape outside the format: {n}x{k}")
        check_artifact(e["packed"], n * k // 2, f"{key} payload")
        check_artifact(e["scales"], 2 * n * (k // FORMAT["group"]), f"{key} scales")

    desc = manifest.get("descriptor")
    require(desc is not None, "the manifest records no descriptor")
    roles_of = None
    if desc is not None:
        require(os.path.exists(desc["path"]) and sha256_file(desc["path"]) == desc["sha256"],
                "the descriptor is missing or no longer matches its digest")
        if os.path.exists(desc["path"]):
            with open(desc["path"]) as handle:
                d = json.load(handle)
            roles_of = (d["num_layers"], d["role_names"])
    covered = set()
    for cell in manifest["precision_map"]:
        key = (cell["layer"], cell["role"])
        require(key not in covered, f"the precision map lists {key} twice")
        covered.add(key)
        require((cell["precision"] == "int4") == (key in seen),
                f"the precision map and the entries disagree about {key}")
    if roles_of is not None:
        for layer in range(roles_of[0]):
            for role in roles_of[1]:
                require((layer, role) in covered, f"the precision map does not cover {(layer, role)}")

    for pair in manifest.get("pairs", []):
        layer = pair["layer"]
        roles = [m["role"] for m in pair["members"]]
        require(roles == list(PAIR_ROLES), f"pair at layer {layer} has members {roles}")
        members = [seen.get((layer, r)) for r in roles]
        if any(m is None for m in members):
            problems.append(f"pair at layer {layer} names a member that has no entry")
            continue
        rows = sum(m["logical_shape"][0] for m in members)
        k = members[0]["logical_shape"][1]
        require(pair["logical_shape"] == [rows, k], f"pair at layer {layer} claims {pair['logical_shape']}")
        for kind in ("packed", "scales"):
            want = b""
            for m in members:
                with open(os.path.join(out_dir, m[kind]["file"]), "rb") as handle:
                    want += handle.read()
            path = os.path.join(out_dir, pair[kind]["file"])
            have = open(path, "rb").read() if os.path.exists(path) else None
            require(have == want, f"pair at layer {layer}'s {kind} is not its members' rows in order")

    if not problems and sample:
        index = read_safetensors_index(source_dir)
        for e in entries[:sample]:
            w = read_bf16_as_f32(index[e["checkpoint_tensor"]])
            if reference:
                packed, scales = _quantize_with(reference, w)
            else:
                p, sc = w4a16.quantize_int4(np.ascontiguousarray(w, dtype=np.float32))
                packed, scales = p.tobytes(), sc.tobytes()
            with open(os.path.join(out_dir, e["packed"]["file"]), "rb") as handle:
                require(handle.read() == packed, f"{e['role']}_{e['layer']} does not re-derive from the source")
            with open(os.path.join(out_dir, e["scales"]["file"]), "rb") as handle:
                require(handle.read() == scales, f"{e['role']}_{e['layer']} scales do not re-derive")
    return problems


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--model-dir")
    ap.add_argument("--desc")
    ap.add_argument("--out-dir")
    ap.add_argument("--limit-layers", type=int)
    ap.add_argument("--verify", metavar="MANIFEST")
    ap.add_argument("--reference", help="a compiled quantizer with --quantize (optional)")
    args = ap.parse_args()
    if args.verify:
        problems = verify(args.verify, args.reference)
        for p in problems:
            print(f"convert: verify: {p}")
        print("convert: verify: ok" if not problems else f"convert: verify: {len(problems)} problem(s)")
        return 1 if problems else 0
    if not (args.model_dir and args.desc and args.out_dir):
        ap.error("--model-dir, --desc and --out-dir are required to convert")
    manifest = convert_checkpoint(args.model_dir, args.desc, args.out_dir, args.limit_layers)
    print(f"convert: {len(manifest['entries'])} entries, {len(manifest['pairs'])} pairs -> "
          f"{os.path.join(args.out_dir, 'weights.manifest.json')}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
