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

--verify audits a written sidecar without trusting what it records (the checks the reference's
--verify makes, scripts/quantize_weights.py:328-460, organised as five passes of this file's
own: header, files, tables, provenance, re-derivation; see the --verify section below).
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
#
# A shard is an 8-byte little-endian header length, a JSON header mapping tensor names to
# {dtype, shape, data_offsets} (offsets relative to the end of the header), then raw bytes. A
# Checkpoint reads every shard's header once, keeps a TensorRef (absolute byte span) per name and
# reads a tensor's bytes only when asked, so a converter run never holds a shard whole.

class TensorRef(tuple):
    """(shard path, dtype, shape, absolute first byte, byte count) of one stored tensor."""

    __slots__ = ()

    def __new__(cls, path, dtype, shape, offset, nbytes):
        return tuple.__new__(cls, (path, dtype, tuple(shape), offset, nbytes))

    path = property(lambda self: self[0])
    dtype = property(lambda self: self[1])
    shape = property(lambda self: self[2])
    offset = property(lambda self: self[3])
    nbytes = property(lambda self: self[4])


def _shard_header(path):
    """The parsed header of one shard and the absolute offset its data region starts at."""
    size = os.path.getsize(path)
    with open(path, "rb") as handle:
        prefix = handle.read(8)
        if len(prefix) != 8:
            raise ConvertError(f"{os.path.basename(path)}: shorter than a safetensors prefix")
        (length,) = struct.unpack("<Q", prefix)
        if 8 + length > size:
            raise ConvertError(f"{os.path.basename(path)}: header of {length} bytes runs past the file")
        header = json.loads(handle.read(length).decode("utf-8"))
    return header, 8 + length, size


class Checkpoint:
    """Every tensor of a directory of safetensors shards, by name (shards in name order).

    Replaces the reference converter's shard index (scripts/quantize_weights.py:75-94) for this
    converter: a name stored by more than one shard, or a byte span outside its shard, is a
    refusal, since either would make the artifact's source ambiguous."""

    def __init__(self, model_dir):
        self.model_dir = model_dir
        self.shards = sorted(f for f in os.listdir(model_dir) if f.endswith(".safetensors"))
        self.refs = {}
        owner = {}
        for shard in self.shards:
            path = os.path.join(model_dir, shard)
            header, base, size = _shard_header(path)
            for name in sorted(k for k in header if k != "__metadata__"):
                if name in owner:
                    raise ConvertError(f"checkpoint tensor {name} is stored by two shards: "
                                       f"{owner[name]} and {shard}")
                lo, hi = header[name]["data_offsets"]
                if not 0 <= lo <= hi or base + hi > size:
                    raise ConvertError(f"{shard}: {name} spans bytes {lo}..{hi}, outside the shard")
                owner[name] = shard
                self.refs[name] = TensorRef(path, header[name]["dtype"], header[name]["shape"],
                                            base + lo, hi - lo)

    def __contains__(self, name):
        return name in self.refs

    def bf16_as_f32(self, name):
        """Tensor `name`, which must be stored as BF16, widened to FP32 (exact)."""
        return read_bf16_as_f32(self.refs[name])


def read_bf16_as_f32(ref):
    """A stored BF16 tensor widened to FP32 (exact: the BF16 bits become the high half)."""
    if ref.dtype != "BF16":
        raise ConvertError(f"only BF16 sources are admitted, got {ref.dtype}")
    count = int(np.prod(ref.shape)) if ref.shape else 1
    if ref.nbytes != 2 * count:
        raise ConvertError(f"{ref.path}: a {list(ref.shape)} BF16 tensor spans {ref.nbytes} bytes")
    with open(ref.path, "rb") as handle:
        handle.seek(ref.offset)
        raw = handle.read(ref.nbytes)
    bits = np.frombuffer(raw, dtype="<u2").astype(np.uint32) << 16
    return bits.view(np.float32).reshape(ref.shape)


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
    ckpt = Checkpoint(model_dir)
    layers, tensor_names = {}, {}
    for layer in range(desc["num_layers"]):
        if desc["layer_ffns"][layer] != "dense" or (limit_layers is not None and layer >= limit_layers):
            continue
        layers[layer] = {}
        for role in ROLES:
            tensor = _role_tensor(templates[names.index(role)], layer)
            if tensor not in ckpt:
                raise ConvertError(f"{tensor} is not in the checkpoint")
            w = ckpt.bf16_as_f32(tensor)
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
#
# An audit of a written sidecar that trusts nothing it records. It runs five passes, each
# appending findings (plain sentences) to one list:
#   1. the header: manifest_version and the frozen FORMAT block;
#   2. the files: every artifact record (entries and pairs alike) against the bytes the shape
#      implies, the bytes recorded, and the file's SHA-256; each file is hashed once;
#   3. the tables: entries unique and inside the tile rule, the precision map a one-to-one cover
#      of the descriptor's (layer, role) grid that marks exactly the entries as int4, every pair
#      [mlpGate, mlpUp] with its members' stacked shape and the hash of their streamed
#      concatenation;
#   4. provenance: the source shards and the descriptor still hash to what was recorded;
#   5. only on a clean audit: a spread sample of entries re-quantized from the source
#      checkpoint, by this library or by a compiled quantizer given as `reference`.

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


def _cell(layer, role):
    return f"layer {layer} {role}"


class _SidecarAudit:
    def __init__(self, manifest_path):
        with open(manifest_path) as handle:
            self.doc = json.load(handle)
        self.root = os.path.dirname(os.path.abspath(manifest_path))
        self.findings = []
        self._hashes = {}

    def note(self, text):
        self.findings.append(text)

    def file_hash(self, rel):
        """SHA-256 of an artifact file under the sidecar's directory, or None when absent."""
        if rel not in self._hashes:
            path = os.path.join(self.root, rel)
            self._hashes[rel] = sha256_file(path) if os.path.isfile(path) else None
        return self._hashes[rel]

    # 1
    def header(self):
        version = self.doc.get("manifest_version")
        if version != MANIFEST_VERSION:
            self.note(f"manifest_version {version!r} is not {MANIFEST_VERSION}, the one this reader knows")
        block = self.doc.get("format") or {}
        for key in FORMAT:
            if block.get(key) != FORMAT[key]:
                self.note(f"format block: {key!r} reads {block.get(key)!r} where the INT4 format "
                          f"fixes {FORMAT[key]!r}")

    # 2
    def files(self):
        group = FORMAT["group"]
        records = []
        for e in self.doc.get("entries", []):
            records.append((f"{_cell(e['layer'], e['role'])}", e, e["logical_shape"]))
        for p in self.doc.get("pairs", []):
            records.append((f"F1 pair of layer {p['layer']}", p, p["logical_shape"]))
        for label, rec, (n, k) in records:
            implied = {"packed": n * k // 2, "scales": 2 * n * (k // group)}
            for kind, want in implied.items():
                art = rec[kind]
                path = os.path.join(self.root, art["file"])
                if not os.path.isfile(path):
                    self.note(f"{label} {kind}: file {art['file']} is absent")
                    continue
                size = os.path.getsize(path)
                if not size == art["bytes"] == want:
                    self.note(f"{label} {kind}: {size} bytes on disk, {art['bytes']} recorded, "
                              f"{want} implied by the shape {n}x{k}")
                if self.file_hash(art["file"]) != art["sha256"]:
                    self.note(f"{label} {kind}: content hash differs from the recorded sha256")

    # 3
    def tables(self, grid):
        from collections import Counter

        entries = {}
        for e in self.doc.get("entries", []):
            key = (e["layer"], e["role"])
            if key in entries:
                self.note(f"{_cell(*key)} is quantized by more than one entry")
            entries[key] = e
            n, k = e["logical_shape"]
            if n % 8 or k % FORMAT["group"]:
                self.note(f"{_cell(*key)}: shape {n}x{k} breaks the tile rule "
                          f"(rows a multiple of 8, K of {FORMAT['group']})")
        cells = Counter()
        for c in self.doc.get("precision_map", []):
            key = (c["layer"], c["role"])
            cells[key] += 1
            if (c["precision"] == "int4") != (key in entries):
                self.note(f"precision_map marks {_cell(*key)} {c['precision']} but the sidecar "
                          f"{'has' if key in entries else 'has no'} INT4 entry for it")
        for key, count in sorted(cells.items()):
            if count > 1:
                self.note(f"precision_map: {_cell(*key)} occurs {count} times")
        for key in grid or ():
            if key not in cells:
                self.note(f"precision_map: no cell for the descriptor's {_cell(*key)}")
        for p in self.doc.get("pairs", []):
            label = f"F1 pair of layer {p['layer']}"
            roles = [m["role"] for m in p["members"]]
            if roles != list(PAIR_ROLES):
                self.note(f"{label}: members are {roles}, the fused kernels need {list(PAIR_ROLES)}")
            parts = [entries.get((p["layer"], r)) for r in roles]
            if None in parts:
                missing = [r for r, e in zip(roles, parts) if e is None]
                self.note(f"{label}: {missing} have no INT4 entry to stack")
                continue
            stacked = [sum(e["logical_shape"][0] for e in parts), parts[0]["logical_shape"][1]]
            if p["logical_shape"] != stacked:
                self.note(f"{label}: logical_shape {p['logical_shape']} but its members stack to {stacked}")
            for kind in ("packed", "scales"):
                have = self.file_hash(p[kind]["file"])
                files = [os.path.join(self.root, e[kind]["file"]) for e in parts]
                if have is None or not all(os.path.isfile(f) for f in files):
                    continue  # already a finding of the file pass
                digest = hashlib.sha256()
                for f in files:
                    with open(f, "rb") as handle:
                        for chunk in iter(lambda: handle.read(1 << 20), b""):
                            digest.update(chunk)
                if digest.hexdigest() != have:
                    self.note(f"{label}: the {kind} file is not the gate rows followed by the up rows")
        return entries

    # 4
    def provenance(self):
        """Returns the descriptor's (layer, role) grid, or None when it cannot be read."""
        source = self.doc["source"]
        for rec in source["files"]:
            path = os.path.join(source["model_dir"], rec["name"])
            if not os.path.isfile(path):
                self.note(f"source checkpoint: shard {rec['name']} is gone")
            elif sha256_file(path) != rec["sha256"]:
                self.note(f"source checkpoint: shard {rec['name']} was modified after conversion")
        desc = self.doc.get("descriptor")
        if desc is None:
            self.note("no descriptor is recorded, so the precision map's cover cannot be checked")
            return None
        if not os.path.isfile(desc["path"]):
            self.note(f"descriptor {desc['path']} is gone")
            return None
        if sha256_file(desc["path"]) != desc["sha256"]:
            self.note(f"descriptor {desc['path']} was modified after conversion")
        with open(desc["path"]) as handle:
            d = json.load(handle)
        return [(layer, role) for layer in range(d["num_layers"]) for role in d["role_names"]]

    # 5
    def rederive(self, entries, reference, sample):
        import w4a16

        ordered = [entries[key] for key in sorted(entries)]
        if not ordered or sample <= 0:
            return
        stride = max(1, len(ordered) // sample)
        ckpt = Checkpoint(self.doc["source"]["model_dir"])
        for e in ordered[::stride][:sample]:
            w = ckpt.bf16_as_f32(e["checkpoint_tensor"])
            if reference:
                packed, scales = _quantize_with(reference, w)
            else:
                p, s = w4a16.quantize_int4(np.ascontiguousarray(w, dtype=np.float32))
                packed, scales = p.tobytes(), s.tobytes()
            for kind, want in (("packed", packed), ("scales", scales)):
                if self.file_hash(e[kind]["file"]) != hashlib.sha256(want).hexdigest():
                    self.note(f"{_cell(e['layer'], e['role'])}: re-quantizing {e['checkpoint_tensor']} "
                              f"gives other {kind} bytes")


def verify(manifest_path, reference=None, sample=2):
    """Audit a written sidecar (the five passes above); returns the findings, empty when clean.

    Covers what the reference's --verify covers (scripts/quantize_weights.py:328-460)."""
    audit = _SidecarAudit(manifest_path)
    audit.header()
    audit.files()
    grid = audit.provenance()
    entries = audit.tables(grid)
    if not audit.findings:
        audit.rederive(entries, reference, sample)
    return audit.findings

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
