"""The prepared-weight loader (glm-flash-rs src/prepared.rs) behind gfr_prepared_*: the format's SHA-256 (FIPS 180-4
known answers, and Python's hashlib), Tensor::extent (the reference's own unit tests, prepared.rs:380-412), the
manifest checks of open_parts (:186-230) and the tree walk (:101-132), and on the GPU: load_selected with per-chunk
hash checks (:270-366), Loaded::pointer (:369-377) and an expert layer run from loaded weights."""
import hashlib
import os

import numpy as np
import pytest

import gfr_moe
import prepared_files as pf


# ---- SHA-256 ---------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("msg,digest", [
    (b"abc", "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"),
    (b"", "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"),
    (b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
     "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"),
    (b"a" * 1000000, "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"),
])
def test_sha256_known_answers(msg, digest):
    assert gfr_moe.sha256_hex(msg) == digest


def test_sha256_matches_hashlib_on_block_edges():
    rng = np.random.default_rng(5)
    for n in (1, 55, 56, 63, 64, 65, 119, 120, 127, 128, 1000, 4096 + 17):
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert gfr_moe.sha256_hex(b) == hashlib.sha256(b).hexdigest(), n


# ---- Tensor::extent: the reference's unit tests (prepared.rs:380-412) -------------------------------------------------
def test_extent_reference_cases():
    assert gfr_moe.tensor_extent("bfloat16", [2, 3], [8, 1], 4) == 30          # strided_extent_includes_offset_and_holes
    with pytest.raises(gfr_moe.GfrError):                                       # reject_integer_overflow
        gfr_moe.tensor_extent("bfloat16", [2, 3], [2 ** 64 - 1, 1], 4)
    with pytest.raises(gfr_moe.GfrError):                                       # reject_rank_mismatch
        gfr_moe.tensor_extent("bfloat16", [2, 3], [8], 4)
    assert gfr_moe.tensor_extent("bfloat16", [0, 3], [8, 1], 4) == 8           # empty_view_does_not_underflow
    with pytest.raises(gfr_moe.GfrError, match="unsupported dtype"):
        gfr_moe.tensor_extent("complex64", [1], [1], 0)


# ---- open / walk / expect / read ---------------------------------------------------------------------------------------
def _model(tmp, chunk=64, mutate=None, tree=None, gaps=3):
    rng = np.random.default_rng(1)
    a = rng.integers(-2 ** 31, 2 ** 31, (4, 6), dtype=np.int64).astype(np.int32)
    b = rng.standard_normal(40).astype(np.float16)
    c = rng.integers(0, 255, 10, dtype=np.uint8)
    storages = [("cuda", a.tobytes()), ("cuda", b.tobytes()), ("cpu", c.tobytes())]
    tree = tree or {"O": "Root", "f": {
        "a": pf.tensor_node(0, "int32", [4, 6]),
        "seq": {"L": [pf.tensor_node(1, "float16", [2, 5], [10, 2], off=3), {"P": 7}]},
        "d": {"D": [["k", pf.tensor_node(1, "float16", [40])], [3, {"U": [pf.tensor_node(2, "uint8", [10], dev="cpu")]}]]},
        "dev": {"dev": "cuda:0"}}}
    return pf.write(str(tmp), storages, tree, chunk=chunk, gaps=gaps, mutate=mutate), (a, b, c)


def test_open_walk_and_read(tmp_path):
    path, (a, b, c) = _model(tmp_path)
    p = gfr_moe.Prepared(path)
    assert p.names() == sorted(['weights.a', 'weights.d["k"]', 'weights.d[3][0]', 'weights.seq[0]'])
    t = p.tensor("weights.seq[0]")
    assert (t.dtype.decode(), t.rank, list(t.shape[:2]), list(t.stride[:2]), t.off, t.cuda) == \
        ("float16", 2, [2, 5], [10, 2], 3, 1)
    assert t.extent_bytes == (3 + 10 + 8 + 1) * 2
    assert p.read_tensor("weights.a") == a.tobytes()
    assert p.read_tensor('weights.d["k"]') == b.tobytes()
    assert p.read_tensor("weights.d[3][0]") == c.tobytes()
    assert p.read_tensor("weights.seq[0]") == b.tobytes()[6:6 + 19 * 2]     # the view's extent past its offset
    assert p.read_tensor("weights.a", 8, 12) == a.tobytes()[8:20]
    with pytest.raises(gfr_moe.GfrError, match="outside extent"):
        p.read_tensor("weights.a", 90, 7)
    p.expect("weights.a", "int32", [4, 6])
    for args, msg in [(("weights.a", "int32", [6, 4]), "unsupported tensor"),
                      (("weights.a", "float32", [4, 6]), "unsupported tensor"),
                      (("weights.seq[0]", "float16", [2, 5]), "noncontiguous"),
                      (("weights.d[3][0]", "uint8", [10]), "unsupported tensor"),      # a cpu tensor
                      (("weights.none", "int32", [1]), "missing tensor")]:
        with pytest.raises(gfr_moe.GfrError, match=msg):
            p.expect(*args)
    p.close()


def _set(path, value):
    def f(m):
        node = m
        for k in path[:-1]:
            node = node[k]
        node[path[-1]] = value
    return f


@pytest.mark.parametrize("mutate,msg", [
    (_set(["format"], 2), "unsupported prepared format"),
    (_set(["chunk"], 0), "invalid chunk size"),
    (_set(["chunk"], 128 * 1024 * 1024 + 1), "invalid chunk size"),
    (lambda m: m["chunk_sha256"].pop(), "chunk hash count"),
    (_set(["file_size"], 5), "chunk hash count|data file size"),
    (_set(["storages", 1, "offset"], 0), "overlapping"),
    (_set(["storages", 0, "nbytes"], 0), "empty/overlapping"),
    (_set(["storages", 2, "nbytes"], 10 ** 6), "outside data file"),
    (_set(["storages", 0, "dev"], "rocm"), "unknown storage device"),
    (_set(["tree", "f", "a", "shape"], [4, 7]), "escapes storage"),
    (_set(["tree", "f", "a", "dev"], "cpu"), "changes device"),
    (_set(["tree", "f", "a", "T"], 9), "missing storage"),
    (_set(["tree", "f", "a"], {"N": [1]}), "NumPy storage"),
    (_set(["tree", "f", "a"], {"f": {}}), "untyped object"),
    (_set(["tree", "f", "a"], {"Q": 1}), "unknown prepared node"),
    (_set(["tree", "f", "a"], {"D": [["only"]]}), "dict pair length"),
    (_set(["tree", "f", "a"], 3), "not an object"),
    (_set(["tree"], {"O": "Root", "f": {}}), "no tensors"),
])
def test_open_rejects(tmp_path, mutate, msg):
    path, _ = _model(tmp_path, mutate=mutate)
    with pytest.raises(gfr_moe.GfrError, match=msg) as e:
        gfr_moe.Prepared(path)
    assert e.value.code == gfr_moe.GFR_EINVAL


def test_open_rejects_bad_json_and_missing_data(tmp_path):
    path, _ = _model(tmp_path)
    with open(path, "a") as f:
        f.write("x")
    with pytest.raises(gfr_moe.GfrError, match="not JSON"):
        gfr_moe.Prepared(path)
    path, _ = _model(tmp_path / "b")
    os.remove(os.path.join(os.path.dirname(path), "data.bin"))
    with pytest.raises(gfr_moe.GfrError, match="cannot open"):
        gfr_moe.Prepared(path)


# ---- GPU: load, hashes, pointers, an expert layer from loaded weights ------------------------------------------------
@pytest.mark.gpu
def test_load_pointer_and_hashes(tmp_path):
    import torch
    path, (a, b, c) = _model(tmp_path, chunk=16)
    p = gfr_moe.Prepared(path)
    nbytes, secs = p.load()
    assert nbytes == a.nbytes + b.nbytes and secs >= 0
    ga = gfr_moe._view(p.pointer("weights.a"), a.shape, torch.int32, "cuda")
    assert np.array_equal(ga.cpu().numpy(), a)
    gb = gfr_moe._view(p.pointer("weights.seq[0]"), (37,), torch.float16, "cuda")   # off 3 elements into storage 1
    assert np.array_equal(gb.cpu().numpy().view(np.uint16), b[3:].view(np.uint16))
    with pytest.raises(gfr_moe.GfrError, match="CPU tensor"):
        p.pointer("weights.d[3][0]")
    # selection: only the storage of weights.a
    p.load(["weights.a"])
    p.pointer("weights.a")
    with pytest.raises(gfr_moe.GfrError, match="not loaded"):
        p.pointer('weights.d["k"]')
    p.close()
    # a corrupted byte inside storage 1 fails the load, but not a selection whose chunks do not hold it
    data = os.path.join(os.path.dirname(path), "data.bin")
    raw = bytearray(open(data, "rb").read())
    pos = 3 + a.nbytes + 3 + 20                      # gaps of 3 bytes before each storage
    raw[pos] ^= 0xFF
    open(data, "wb").write(raw)
    p = gfr_moe.Prepared(path)
    with pytest.raises(gfr_moe.GfrError, match=f"weight hash mismatch in chunk {pos // 16}"):
        p.load()
    p.load(["weights.a"])
    assert np.array_equal(gfr_moe._view(p.pointer("weights.a"), a.shape, torch.int32, "cuda").cpu().numpy(), a)
    p.close()


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 64])
def test_moe_layer_from_prepared_weights(tmp_path, rows):
    """One decode token and a 64-row window through Moe with the loaded weights: bit-identical to the same layer run
    from the tensors that were written."""
    import torch
    import synth
    E, D, N, topk, bits = 16, 256, 512, 2, 3
    w = synth.experts(E + 1, D, N, bits, seed=17)
    names = ("gt", "ut", "dt", "suh_g", "suh_u", "suh_d", "svh_g", "svh_u", "svh_d")
    host = {n: getattr(w, n).cpu().numpy() for n in names}
    path = pf.write_experts(str(tmp_path), [host, host])
    p = gfr_moe.Prepared(path)
    p.load(["weights.layers[1]."])
    wl = p.experts(1)
    assert (wl.experts, wl.hidden, wl.inter, wl.bits) == (E + 1, D, N, bits)
    with pytest.raises(gfr_moe.GfrError, match="not loaded"):
        p.experts(0)
    x = synth.activations(rows, D, 3)
    lg = synth.logits(rows, E, 4)
    outs = []
    for weights in (w, wl):
        m = gfr_moe.Moe(D, N, E, topk, rows)
        m.run(weights, x, lg, rows)
        torch.cuda.synchronize()
        outs.append(m.output.clone().cpu())
    assert torch.equal(outs[0], outs[1])
    p.close()


def test_package_writer_round_trip(tmp_path):
    """gfr_moe.write_prepared (the bench's writer) produces a model the loader opens, with the expert paths and bytes."""
    rng = np.random.default_rng(9)
    names = ("gt", "ut", "dt", "suh_g", "suh_u", "suh_d", "svh_g", "svh_u", "svh_d")
    layers = []
    for _ in range(2):
        layers.append({n: rng.integers(-2 ** 31, 2 ** 31, (3, 2, 3, 24), dtype=np.int64).astype(np.int32)
                       if n in ("gt", "ut", "dt") else rng.standard_normal((3, 32)).astype(np.float16) for n in names})
    p = gfr_moe.Prepared(gfr_moe.write_prepared(str(tmp_path), layers, chunk=700))
    for L, layer in enumerate(layers):
        for n in names:
            path = f"weights.layers[{L}].moe.experts.{n}"
            assert p.read_tensor(path) == layer[n].tobytes()
            t = p.tensor(path)
            assert list(t.shape[:t.rank]) == list(layer[n].shape)
    p.close()


def test_shared_fp8_tensors_round_trip(tmp_path):
    """write_prepared carries the FP8 shared expert as weights.layers[L].moe.shared.{gu,down}.{weight,scale}
    (float8_e4m3fn bytes, bfloat16 scales, the shapes moe.rs:136-161 reads); the reader finds them and returns their
    bytes, without a GPU."""
    import torch
    import synth
    small = synth.experts(2, 512, 256, 4, seed=3, device="cpu")
    sw = synth.fp8_shared(512, 256, seed=5, device="cpu")
    p = gfr_moe.Prepared(gfr_moe.write_prepared(str(tmp_path / "p"), [small], shared=[sw]))
    stem = "weights.layers[0].moe.shared."
    assert sorted(n for n in p.names() if n.startswith(stem)) == [
        stem + "down.scale", stem + "down.weight", stem + "gu.scale", stem + "gu.weight"]
    p.expect(stem + "gu.weight", "float8_e4m3fn", [512, 512])
    p.expect(stem + "gu.scale", "bfloat16", [512])
    p.expect(stem + "down.weight", "float8_e4m3fn", [512, 256])
    p.expect(stem + "down.scale", "bfloat16", [512])
    assert p.read_tensor(stem + "down.weight") == sw.down.numpy().tobytes()
    assert p.read_tensor(stem + "gu.scale") == sw.gu_scale.view(torch.int16).numpy().tobytes()
