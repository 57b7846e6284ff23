"""The safetensors expert store (libdsv4_expert_store.so): header and index
parsing, host reads and error paths on the CPU; device loads into the routed
kernels' expert-major tensors on the GPU. Fixtures are written with the
safetensors package (the format's own writer), plus hand-made files for
parser edge cases."""
from __future__ import annotations

import ctypes
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oracle import mx
from runtime import synth
from tests.conftest import PKG

LIB = os.path.join(PKG, "kernel", "expert-store", "libdsv4_expert_store.so")

E, K, H, O = 4, 512, 256, 384   # experts per layer, w1/w3 [H, K], w2 [O, H]


def _store_mod():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run __graft_entry__.build() first")
    from runtime import expert_store
    return expert_store


def _experts(layer):
    """Seeded MXFP4 experts of one layer: {proj: (packed [E, rows, cols/2], scale [E, rows, cols/32])}."""
    out = {}
    for m, (proj, rows, cols) in enumerate((("w1", H, K), ("w3", H, K), ("w2", O, H))):
        out[proj] = synth.mxfp4_weight(9700 + 10 * layer + m, rows, cols, E)
    return out


def _tensors(layer, experts):
    t = {}
    for proj, (p, s) in experts.items():
        for e in range(E):
            base = f"layers.{layer}.ffn.experts.{e}.{proj}"
            t[base + ".weight"] = torch.from_numpy(p[e].view(np.int8).copy())
            t[base + ".scale"] = torch.from_numpy(s[e].copy()).view(torch.float8_e8m0fnu)
    t[f"layers.{layer}.attn_norm.weight"] = torch.arange(16, dtype=torch.float32).to(torch.bfloat16)
    t[f"layers.{layer}.attn.attn_sink"] = torch.arange(8, dtype=torch.float32) / 8 - 0.5
    t[f"layers.{layer}.attn.wq_a.weight"] = torch.from_numpy(
        synth.fp8_weight(9800 + layer, 128, 256)[0].copy()).view(torch.float8_e4m3fn)
    return t


@pytest.fixture(scope="module")
def snapshot(tmp_path_factory):
    """Two layers in two shards with an index, as a Hugging Face snapshot."""
    d = tmp_path_factory.mktemp("snap")
    experts = {L: _experts(L) for L in (0, 1)}
    weight_map = {}
    for L in (0, 1):
        shard = f"model-{L + 1:05d}-of-00002.safetensors"
        t = _tensors(L, experts[L])
        save_file(t, str(d / shard), metadata={"format": "pt"})
        weight_map.update({k: shard for k in t})
    with open(d / "model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": weight_map}, f)
    return d, experts, weight_map


def test_index_snapshot_info_and_host_reads(snapshot):
    es = _store_mod()
    d, experts, weight_map = snapshot
    with es.ExpertStore(str(d)) as st:
        assert len(st) == len(weight_map)
        for L in (0, 1):
            for proj, (p, s) in experts[L].items():
                for e in range(E):
                    base = f"layers.{L}.ffn.experts.{e}.{proj}"
                    dt, shape, nb = st.info(base + ".weight")
                    assert (dt, shape, nb) == ("I8", p[e].shape, p[e].size)
                    assert st.info(base + ".scale") == ("F8_E8M0", s[e].shape, s[e].size)
                    assert np.array_equal(st.read(base + ".weight").view(np.uint8), p[e])
                    assert np.array_equal(st.read(base + ".scale"), s[e])
            norm = st.read(f"layers.{L}.attn_norm.weight")
            assert norm.dtype == np.uint16 and np.array_equal(
                norm, torch.arange(16, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
            assert np.array_equal(st.read(f"layers.{L}.attn.attn_sink"), np.arange(8, dtype=np.float32) / 8 - 0.5)
            assert st.info(f"layers.{L}.attn.wq_a.weight")[:2] == ("F8_E4M3", (128, 256))
        with pytest.raises(KeyError):
            st.info("layers.7.ffn.experts.0.w1.weight")


def test_single_file_and_single_model_dir(tmp_path):
    es = _store_mod()
    t = _tensors(3, _experts(3))
    save_file(t, str(tmp_path / "model.safetensors"))
    for path in (tmp_path / "model.safetensors", tmp_path):
        with es.ExpertStore(str(path)) as st:
            assert len(st) == len(t)
            name = "layers.3.ffn.experts.2.w2.weight"
            assert np.array_equal(st.read(name), t[name].numpy())


def _raw_file(path, header: bytes, payload: bytes):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header)))
        f.write(header)
        f.write(payload)


def test_parser_escapes_metadata_and_padding(tmp_path):
    """Names with JSON escapes (quote, backslash, \\u00e9, a surrogate pair),
    nested metadata, numbers in exponent form in the metadata, and trailing
    space padding (as the safetensors writer pads to 8 bytes)."""
    es = _store_mod()
    names = ['a"b', "c\\d", "café", "smile\U0001F600"]
    hdr = {"__metadata__": {"note": "x", "n": "1e3"}}
    payload = b""
    for i, n in enumerate(names):
        hdr[n] = {"dtype": "U8", "shape": [2, 3], "data_offsets": [6 * i, 6 * i + 6]}
        payload += bytes(range(10 * i, 10 * i + 6))
    text = json.dumps(hdr, ensure_ascii=True).encode() + b"   "
    _raw_file(tmp_path / "x.safetensors", text, payload)
    with es.ExpertStore(str(tmp_path / "x.safetensors")) as st:
        assert len(st) == len(names)
        for i, n in enumerate(names):
            assert st.info(n) == ("U8", (2, 3), 6)
            assert np.array_equal(st.read(n).reshape(-1), np.arange(10 * i, 10 * i + 6, dtype=np.uint8))


@pytest.mark.parametrize("case", ["bad json", "offsets past end", "size mismatch", "short file",
                                  "index names a missing shard", "index name not in shard"])
def test_open_rejects_malformed_snapshots(tmp_path, case):
    es = _store_mod()
    good = json.dumps({"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}).encode()
    path = tmp_path / "m.safetensors"
    if case == "bad json":
        _raw_file(path, good[:-1] + b",}", bytes(8))
    elif case == "offsets past end":
        _raw_file(path, json.dumps({"t": {"dtype": "U8", "shape": [16], "data_offsets": [0, 16]}}).encode(), bytes(8))
    elif case == "size mismatch":
        _raw_file(path, json.dumps({"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}).encode(), bytes(8))
    elif case == "short file":
        path.write_bytes(b"\x10\x00\x00")
    else:
        _raw_file(path, good, bytes(8))
        wm = {"t": "m.safetensors", "u": "other.safetensors"} if case == "index names a missing shard" \
            else {"t": "m.safetensors", "u": "m.safetensors"}
        (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
        path = tmp_path
    with pytest.raises(RuntimeError):
        es.ExpertStore(str(path))


def test_mutated_headers_are_parsed_or_rejected(tmp_path):
    """Seeded byte flips, deletions, insertions of JSON punctuation, truncations
    and wrong header lengths of a valid file: every open either fails cleanly
    or yields tensors whose reads stay inside the file (no crash, no read past
    a tensor's bytes). The same mutations ran against an ASan + UBSan host
    build of the library with no finding."""
    import random

    es = _store_mod()
    hdr = {"__metadata__": {"format": "pt", "k\\u00e9y": 'v"q'},
           "w": {"dtype": "I8", "shape": [4, 16], "data_offsets": [0, 64]},
           "s": {"dtype": "F8_E8M0", "shape": [4, 1], "data_offsets": [64, 68]},
           "a\U0001F600b": {"dtype": "BF16", "shape": [2], "data_offsets": [68, 72]}}
    text = json.dumps(hdr, ensure_ascii=True).encode()
    rng = random.Random(20240)
    path = tmp_path / "m.safetensors"
    opened = 0
    for _ in range(400):
        h = bytearray(text)
        for _ in range(rng.randint(1, 6)):
            op = rng.random()
            if op < 0.4 and h:
                h[rng.randrange(len(h))] = rng.randrange(256)
            elif op < 0.6 and h:
                del h[rng.randrange(len(h))]
            elif op < 0.8:
                h.insert(rng.randrange(len(h) + 1), rng.choice(b'{}[]",:\\0123456789eE+-.tfnu'))
            else:
                h = h[:rng.randrange(len(h) + 1)]
        payload = bytes(rng.randrange(256) for _ in range(rng.choice([0, 10, 72, 100])))
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", len(h) if rng.random() < 0.9 else rng.randrange(2 * len(h) + 10)))
            f.write(bytes(h))
            f.write(payload)
        try:
            st = es.ExpertStore(str(path))
        except RuntimeError:
            continue
        opened += 1
        with st:
            for name in ("w", "s", "a\U0001F600b"):
                try:
                    _, _, nbytes = st.info(name)
                except (KeyError, RuntimeError):
                    continue
                assert 0 <= nbytes <= len(payload)
                assert st.read(name).nbytes == nbytes
    assert opened > 0   # some mutations (e.g. in the metadata) leave a valid file


def test_read_capacity_and_argument_errors(snapshot):
    es = _store_mod()
    d, experts, _ = snapshot
    lib = ctypes.CDLL(LIB)
    lib.dsv4_store_open.restype = ctypes.c_void_p
    lib.dsv4_store_open.argtypes = [ctypes.c_char_p]
    lib.dsv4_store_read.restype = ctypes.c_int
    lib.dsv4_store_read.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64]
    lib.dsv4_store_close.argtypes = [ctypes.c_void_p]
    lib.dsv4_store_load_experts.restype = ctypes.c_int
    lib.dsv4_store_load_experts.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_int,
                                            ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    h = lib.dsv4_store_open(str(d).encode())
    assert h
    buf = np.zeros(64, np.uint8)
    p = buf.ctypes.data_as(ctypes.c_void_p)
    name = b"layers.0.ffn.experts.0.w1.scale"   # 256 x 16 bytes
    assert lib.dsv4_store_read(h, name, p, 64) == -3
    assert lib.dsv4_store_read(h, b"nope", p, 64) == -1
    assert lib.dsv4_store_read(None, name, p, 64) == -2
    # argument checks precede any HIP call
    fake = ctypes.c_void_p(16)
    assert lib.dsv4_store_load_experts(h, 0, b"w4", 4, fake, 1 << 20, fake, 1 << 20, None, None, None) == -2
    assert lib.dsv4_store_load_experts(h, 0, b"w1", 0, fake, 1 << 20, fake, 1 << 20, None, None, None) == -2
    assert lib.dsv4_store_load_experts(h, 0, b"w1", 9, fake, 1 << 20, fake, 1 << 20, None, None, None) == -1
    assert lib.dsv4_store_load_experts(h, 0, b"w1", 4, fake, 100, fake, 1 << 20, None, None, None) == -3
    lib.dsv4_store_close(h)


def test_load_experts_wrong_dtype_is_rejected(tmp_path):
    """An expert whose packed weight is stored as U8 instead of I8 (-4), before any copy."""
    es = _store_mod()
    t = _tensors(0, _experts(0))
    t["layers.0.ffn.experts.1.w3.weight"] = t["layers.0.ffn.experts.1.w3.weight"].view(torch.uint8)
    save_file(t, str(tmp_path / "model.safetensors"))
    lib = ctypes.CDLL(LIB)
    lib.dsv4_store_open.restype = ctypes.c_void_p
    lib.dsv4_store_open.argtypes = [ctypes.c_char_p]
    lib.dsv4_store_load_experts.restype = ctypes.c_int
    lib.dsv4_store_load_experts.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_int,
                                            ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.dsv4_store_close.argtypes = [ctypes.c_void_p]
    h = lib.dsv4_store_open(str(tmp_path).encode())
    fake = ctypes.c_void_p(16)
    assert lib.dsv4_store_load_experts(h, 0, b"w3", 4, fake, 1 << 20, fake, 1 << 20, None, None, None) == -4
    lib.dsv4_store_close(h)


@pytest.mark.gpu
def test_load_layer_to_hbm_and_run_the_routed_layer(snapshot, device):
    """load_layer fills the expert-major tensors byte for byte; the routed
    layer run on them matches the oracle on the source experts."""
    es = _store_mod()
    from runtime import mxfp4_grouped_gemv_binding as gb
    from tests.gpu_util import announce, assert_close, dev_bf16, dev_f32, host_bits

    d, experts, _ = snapshot
    announce(f"expert store: load 2 layers x {E} experts, routed layer on layer 1")
    with es.ExpertStore(str(d)) as st:
        for L in (0, 1):
            w = st.load_layer(L, device, n_experts=E)
            for proj, mats in (("w1", w.W1), ("w3", w.W3), ("w2", w.W2)):
                p, s = experts[L][proj]
                assert np.array_equal(mats["packed"].cpu().numpy(), p), f"layer {L} {proj} packed"
                assert np.array_equal(mats["scale"].cpu().numpy(), s), f"layer {L} {proj} scale"
        norm = st.load_tensor("layers.1.attn_norm.weight", device, torch.bfloat16)
        assert torch.equal(norm.cpu(), torch.arange(16, dtype=torch.float32).to(torch.bfloat16))
    T, topk = 3, 2
    x = synth.normal_bf16(9900, (T, K))
    ids, wts = mx.route_sigmoid_topk(synth.gating_logits(9901, T, E), topk)
    out = gb.mxfp4_moe_grouped_gemv(dev_bf16(x, device), w.W1, w.W3, w.W2,
                                    torch.from_numpy(ids).to(device), dev_f32(wts, device))

    def fn(e):
        return tuple((experts[1][proj][0][e], experts[1][proj][1][e]) for proj in ("w1", "w3", "w2"))

    assert_close(host_bits(out), mx.moe_layer(x, fn, ids, wts, O), "routed layer on loaded experts")
