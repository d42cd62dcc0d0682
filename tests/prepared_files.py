"""Writer of the reference's prepared weight format (glm-flash-rs src/prepared.rs:15-40, 101-132) for the loader
tests: a JSON manifest {format, file_size, chunk, chunk_sha256, storages, tree, key} next to data.bin.

`storages` is a list of (dev, bytes) placed one after another (optionally with gaps); `tensors` maps a tree position
to a tensor node. Hashes come from Python's hashlib, independently of the library's own SHA-256."""
import hashlib
import json
import os


def tensor_node(storage, dtype, shape, stride=None, off=0, dev="cuda"):
    if stride is None:
        stride, acc = [], 1
        for n in reversed(shape):
            stride.insert(0, acc)
            acc *= n
    return {"T": storage, "dtype": dtype, "shape": list(shape), "stride": list(stride), "off": off, "dev": dev}


def experts_tree(layers, cfg=None):
    """Root object with layers[L].moe.experts.{name: node} (the paths experts.rs:467 resolves)."""
    return {"O": "tensorfold.families.glm5_next.cuda.weights:Weights",
            "f": {"cfg": {"O": "Cfg", "f": {k: {"P": v} for k, v in (cfg or {"hidden": 0}).items()}},
                  "layers": {"L": [{"O": "Layer", "f": {"moe": {"O": "Moe", "f": {
                      "experts": {"O": "Experts", "f": nodes}}}}} for nodes in layers]}}}


def write(directory, storages, tree, chunk=4096, gaps=0, key=None, mutate=None):
    """Write manifest.json + data.bin; returns the manifest path. `mutate(manifest)` may edit the manifest dict
    before it is written (the malformed-manifest tests)."""
    os.makedirs(directory, exist_ok=True)
    data = bytearray()
    entries = []
    for dev, blob in storages:
        data += b"\x5a" * gaps
        entries.append({"offset": len(data), "nbytes": len(blob), "dev": dev})
        data += bytes(blob)
    hashes = [hashlib.sha256(bytes(data[i:i + chunk])).hexdigest() for i in range(0, len(data), chunk)]
    m = {"format": 1, "file_size": len(data), "chunk": chunk, "chunk_sha256": hashes, "storages": entries,
         "tree": tree, "key": key or {"rank": 0, "world": 1, "model": "synthetic"}}
    if mutate:
        mutate(m)
    with open(os.path.join(directory, "data.bin"), "wb") as f:
        f.write(data)
    path = os.path.join(directory, "manifest.json")
    with open(path, "w") as f:
        json.dump(m, f)
    return path


def write_experts(directory, layers, chunk=1 << 20):
    """One storage per tensor; `layers` is a list of dicts name -> numpy array (int32 trellis, float16 scales)."""
    storages, nodes = [], []
    dt = {"int32": "int32", "float16": "float16"}
    for tensors in layers:
        n = {}
        for name, arr in tensors.items():
            n[name] = tensor_node(len(storages), dt[str(arr.dtype)], arr.shape)
            storages.append(("cuda", arr.tobytes()))
        nodes.append(n)
    return write(directory, storages, experts_tree(nodes), chunk=chunk, gaps=64)
