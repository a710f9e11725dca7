"""The `.hypno` model reader (hypno_hip_model_*, loader.rs / format.rs).

CPU tests open files host-only (no device call) and compare the library's
parse with the oracle restatement (oracle/hypno_format.py) on the reference's
own loader-test file, random valid files, every truncation of a file and
targeted corruptions.  GPU tests check that the uploaded payloads are the
file's bytes exactly and that decode GEMVs driven from the loaded model match
the CPU oracle."""
import ctypes
import os
import random
import re
import struct

import numpy as np
import pytest

from oracle import hypno_format as hf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FIXTURE = os.path.join(ROOT, "tests", "golden", "loader_test.hypno")


@pytest.fixture(scope="module")
def hk():
    import hypno_amd
    return hypno_amd


def _write(tmp_path, data: bytes, name="m.hypno") -> str:
    p = os.path.join(str(tmp_path), name)
    with open(p, "wb") as f:
        f.write(data)
    return p


def _lib_outcome(hk, path):
    """('ok', manifest-as-tuples) or (FormatError kind, fields) from the library."""
    try:
        m = hk.HypnoModel.open(path, device=False)
    except hk.FormatError as e:
        msg = str(e)
        pats = [("BufferTooShort", r"buffer too short: needed (\d+) bytes, got (\d+)"),
                ("InvalidMagic", r"invalid magic bytes"),
                ("UnsupportedVersion", r"unsupported format version (\d+)"),
                ("Utf8", r"UTF-8 error: invalid utf-8 at byte (\d+)"),
                ("UnknownDType", r"unknown dtype code: (\d+)"),
                ("InvalidOffset", r"invalid tensor offset (\d+): out of file bounds \((\d+)\)")]
        for kind, pat in pats:
            mm = re.search(pat, msg)
            if mm:
                return kind, tuple(int(g) for g in mm.groups())
        raise AssertionError(f"unrecognised error message: {msg}")
    with m:
        man = m.manifest
        out = (man.header.version, man.header.metadata_kv_count, man.header.tensor_count,
               [(kv.key, kv.value) for kv in man.metadata],
               [(t.name, t.shape, int(t.dtype), t.offset, t.data_len) for t in man.tensors],
               [bytes(m.get_tensor_data(t.name)[0]) for t in man.tensors])
    return "ok", out


def _oracle_outcome(data: bytes):
    try:
        man = hf.read(data)
    except hf.FormatErr as e:
        fields = () if e.kind == "InvalidMagic" else tuple(int(f) for f in e.fields)
        return e.kind, fields
    # get_tensor_data returns the first tensor with that name (loader.rs:139-149)
    first = {}
    for t in man.tensors:
        first.setdefault(t.name, t)
    return "ok", (man.version, man.metadata_kv_count, man.tensor_count, man.metadata,
                  [(t.name, t.shape, t.dtype, t.offset, t.data_len) for t in man.tensors],
                  [data[first[t.name].offset:first[t.name].offset + first[t.name].data_len]
                   for t in man.tensors])


# --- the oracle against the reference's own tests ------------------------------------

def test_oracle_reads_reference_loader_test_file():
    """Assertions of test_open_and_read (loader.rs:294-319) on its own file."""
    data = open(FIXTURE, "rb").read()
    man = hf.read(data)
    assert (man.metadata_kv_count, man.tensor_count) == (2, 2)
    md = dict(man.metadata)
    assert md["architecture"] == "llama" and md["hidden_size"] == "64"
    w, q = man.tensors
    assert (w.name, w.dtype, w.data_len) == ("weight", 0, 256)
    floats = np.frombuffer(data[w.offset:w.offset + w.data_len], np.float32)
    assert floats.size == 64 and abs(floats[0]) < 1e-3 and abs(floats[63] - 63.0) < 1e-3
    assert (q.name, q.dtype, q.data_len) == ("qweight", 3, 18)


def test_oracle_writer_layout():
    """Converter rules: Q4_0 of 8192 elements is 4608 bytes (sft_convert.rs:452-456),
    small tensors stay FP32 (sft_convert.rs:11-17), payloads start on 64-byte
    boundaries after a data start rounded up to 64 (sft_convert.rs:137-168)."""
    assert hf.data_bytes(3, 8192) == 4608 and hf.data_bytes(2, 8192) == 8704
    assert hf.data_bytes(3, 33) == 36 and hf.data_bytes(1, 5) == 10
    assert hf.effective_dtype(3, 4096) == 0 and hf.effective_dtype(3, 4097) == 3
    assert hf.effective_dtype(1, 64) == 1
    tensors = [("a.weight", (64, 128), 3, bytes(range(256)) * 18),
               ("b.norm", (7,), 0, b"\x01" * 28),
               ("c", (3,), 1, b"\x02" * 6)]
    data = hf.write([("architecture", "llama"), ("weight_layout", "row_major")], tensors)
    man = hf.read(data)
    table_end = 16 + sum(8 + len(k) + len(v) for k, v in man.metadata) + sum(
        4 + len(t.name) + 4 + 8 * t.ndim + 20 for t in man.tensors)
    assert man.tensors[0].offset == (table_end + 63) // 64 * 64
    for t, (name, shape, dtype, payload) in zip(man.tensors, tensors):
        assert t.offset % 64 == 0
        assert (t.name, t.shape, t.dtype, t.data_len) == (name, shape, dtype, len(payload))
        assert data[t.offset:t.offset + t.data_len] == payload
    assert len(data) % 64 == 0


# --- the library against the oracle (host-only: no device) ----------------------------

def test_library_reads_reference_loader_test_file(hk):
    with hk.HypnoModel.open(FIXTURE, device=False) as m:
        assert m.manifest.header.metadata_kv_count == 2
        assert m.manifest.header.tensor_count == 2
        assert m.get_metadata("architecture") == "llama"
        assert m.get_metadata("hidden_size") == "64"
        assert m.get_metadata("vocab_size") is None
        data, dtype = m.get_tensor_data("weight")
        assert dtype == hk.DType.FP32
        floats = np.frombuffer(bytes(data), np.float32)
        assert floats.size == 64 and abs(floats[0]) < 1e-3 and abs(floats[63] - 63.0) < 1e-3
        data, dtype = m.get_tensor_data("qweight")
        assert dtype == hk.DType.Q4_0 and len(data) == 18
        assert m.get_tensor_data("missing") is None and m.find_tensor("missing") is None
        assert not m.is_col_major()
    assert _lib_outcome(hk, FIXTURE) == _oracle_outcome(open(FIXTURE, "rb").read())


def _random_file(rng: random.Random) -> bytes:
    words = ["model", "layers", "0", "self_attn", "q_proj", "weight", "mlp", "норм", "重み", "x"]
    md = [("architecture", "LlamaForCausalLM")]
    for _ in range(rng.randrange(0, 6)):
        md.append(("_".join(rng.choices(words, k=rng.randrange(1, 4))),
                   "".join(rng.choices("abc019é€😀 ", k=rng.randrange(0, 20)))))
    tensors = []
    for i in range(rng.randrange(0, 7)):
        ndim = rng.randrange(0, 4)
        shape = tuple(rng.randrange(1, 9) for _ in range(ndim))
        dtype = rng.randrange(0, 4)
        n = 1
        for d in shape:
            n *= d
        payload = bytes(rng.randrange(256) for _ in range(hf.data_bytes(dtype, n)))
        tensors.append((".".join(rng.choices(words, k=3)) + f".{i}", shape, dtype, payload))
    return hf.write(md, tensors)


def test_random_files_match_oracle(hk, tmp_path):
    rng = random.Random(1234)
    for i in range(40):
        data = _random_file(rng)
        path = _write(tmp_path, data)
        assert _lib_outcome(hk, path) == _oracle_outcome(data), f"file {i}"


def test_every_truncation_matches_oracle(hk, tmp_path):
    data = hf.write([("k", "v"), ("hidden_size", "64")],
                    [("w", (2, 64), 3, bytes(range(72)) * 1), ("n", (3,), 0, b"\x00" * 12)])
    kinds = set()
    for cut in range(len(data) + 1):
        path = _write(tmp_path, data[:cut])
        got, want = _lib_outcome(hk, path), _oracle_outcome(data[:cut])
        assert got == want, f"prefix of {cut} bytes"
        kinds.add(got[0])
    assert kinds == {"BufferTooShort", "InvalidOffset", "ok"}


def _corrupt(data: bytes, pos: int, new: bytes) -> bytes:
    return data[:pos] + new + data[pos + len(new):]


def test_corruptions_match_oracle(hk, tmp_path):
    base = hf.write([("kk", "vvvv")], [("name", (32,), 3, bytes(18))])
    kv_key = 16 + 4                       # first key byte
    kv_val = kv_key + 2 + 4               # first value byte
    name = kv_val + 4 + 4                 # first tensor-name byte
    dtype_pos = name + 4 + 4 + 8
    off_pos = dtype_pos + 4
    cases = {
        "magic": _corrupt(base, 0, b"GGUF"),
        "version": _corrupt(base, 4, struct.pack("<I", 2)),
        "dtype": _corrupt(base, dtype_pos, struct.pack("<I", 4)),
        "offset": _corrupt(base, off_pos, struct.pack("<Q", len(base) + 1)),
        "len": _corrupt(base, off_pos + 8, struct.pack("<Q", len(base))),
        "wrap": _corrupt(base, off_pos + 8, struct.pack("<Q", 2 ** 64 - 8)),
        "key_overlong": _corrupt(base, kv_key, b"\xc0\xaf"),
        "val_surrogate": _corrupt(base, kv_val, b"\xed\xa0\x80"),
        "val_truncated": _corrupt(base, kv_val + 2, b"\xe2\x82"),
        "name_above_max": _corrupt(base, name, b"\xf4\x90\x80\x80"),
        "name_past_end": _corrupt(base, name - 4, struct.pack("<I", 1 << 20)),
        "kv_count": _corrupt(base, 8, struct.pack("<I", 0xFFFFFFFF)),
        "tensor_count": _corrupt(base, 12, struct.pack("<I", 0xFFFF)),
        "ndim": _corrupt(base, name + 4, struct.pack("<I", 0x7FFFFFFF)),
    }
    want_kind = {"magic": "InvalidMagic", "version": "UnsupportedVersion",
                 "dtype": "UnknownDType", "offset": "InvalidOffset", "len": "InvalidOffset",
                 "wrap": "InvalidOffset", "key_overlong": "Utf8", "val_surrogate": "Utf8",
                 "val_truncated": "Utf8", "name_above_max": "Utf8",
                 "name_past_end": "BufferTooShort", "kv_count": "BufferTooShort",
                 "tensor_count": "BufferTooShort", "ndim": "BufferTooShort"}
    for label, data in cases.items():
        got = _lib_outcome(hk, _write(tmp_path, data))
        assert got == _oracle_outcome(data), label
        assert got[0] == want_kind[label], label
    assert _lib_outcome(hk, _write(tmp_path, b"")) == ("BufferTooShort", (16, 0))


def test_lookup_semantics(hk, tmp_path):
    data = hf.write([("weight_layout", "col_major"), ("weight_layout", "row_major"),
                     ("a", "1"), ("a", "2")],
                    [("t", (1,), 0, b"\x01\x00\x00\x00"), ("t", (2,), 1, b"\x02\x00\x03\x00")])
    with hk.HypnoModel.open(_write(tmp_path, data), device=False) as m:
        assert m.is_col_major()                 # first weight_layout wins (loader.rs:158-168)
        assert m.get_metadata("a") == "1"
        t = m.find_tensor("t")
        assert (t.shape, t.dtype) == ((1,), hk.DType.FP32)
        assert bytes(m.get_tensor_data("t")[0]) == b"\x01\x00\x00\x00"
    data = hf.write([("weight_layout", "row_major")], [])
    with hk.HypnoModel.open(_write(tmp_path, data), device=False) as m:
        assert not m.is_col_major() and m.manifest.tensors == []


def test_open_errors(hk, tmp_path):
    with pytest.raises(FileNotFoundError):
        hk.HypnoModel.open(os.path.join(str(tmp_path), "nope.hypno"), device=False)
    with pytest.raises(OSError):
        hk.HypnoModel.open(str(tmp_path), device=False)  # a directory
    from hypno_amd import _lib
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.hypno_hip_model_open(None, 1, ctypes.byref(h)) == 22
    assert lib.hypno_hip_model_open(FIXTURE.encode(), 2, ctypes.byref(h)) == 22
    assert lib.hypno_hip_model_close(None) == 22
    assert lib.hypno_hip_model_is_col_major(None) == 0


# --- device residency ----------------------------------------------------------------

def _hip():
    for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6",
                 "/opt/rocm/lib/libamdhip64.so"):
        try:
            h = ctypes.CDLL(name)
            h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
            return h
        except OSError:
            continue
    raise RuntimeError("libamdhip64 not found")


def _device_bytes(hip, ptr: int, n: int) -> bytes:
    out = ctypes.create_string_buffer(n)
    assert hip.hipMemcpy(out, ctypes.c_void_p(ptr), n, 2) == 0  # hipMemcpyDeviceToHost
    return out.raw


@pytest.mark.gpu
def test_upload_is_byte_exact(hk, tmp_path):
    rng = np.random.default_rng(7)
    big = rng.integers(0, 256, 40 * 1024 * 1024 + 18 * 5, dtype=np.uint8).tobytes()  # 3 pieces
    tensors = [("embed", (5, 7), 0, rng.integers(0, 256, 140, dtype=np.uint8).tobytes()),
               ("big", (len(big) // 18 * 32,), 3, big),
               ("empty", (0,), 0, b""),
               ("odd16", (33,), 1, rng.integers(0, 256, 66, dtype=np.uint8).tobytes())]
    data = hf.write([("architecture", "llama")], tensors)
    path = _write(tmp_path, data)
    print(f"upload test: {len(data)} bytes", flush=True)
    hip = _hip()
    with hk.HypnoModel.open(path) as m:
        for name, _, dtype, payload in tensors:
            ptr, n, dt = m.device_tensor(name)
            t = m.find_tensor(name)
            assert n == len(payload) and int(dt) == dtype
            if n == 0:
                assert ptr == 0
                continue
            assert ptr % 64 == t.offset % 64
            assert _device_bytes(hip, ptr, n) == payload, name


@pytest.mark.gpu
def test_decode_layer_from_loaded_model(hk, orc, tmp_path):
    """One TinyLlama-1.1B layer written as a .hypno file, loaded to HBM, and
    its seven Q4_0 GEMVs run from the model's device pointers through the C ABI
    (one plan launch) against the CPU oracle on the mapped host bytes."""
    import torch
    from hypno_amd import _lib
    shapes = {"q_proj": (2048, 2048), "k_proj": (256, 2048), "v_proj": (256, 2048),
              "o_proj": (2048, 2048), "gate_proj": (5632, 2048), "up_proj": (5632, 2048),
              "down_proj": (2048, 5632)}
    tensors = [("model.layers.0.input_layernorm.weight", (2048,), 0,
                np.ones(2048, np.float32).tobytes())]
    for i, (nm, (n, m)) in enumerate(shapes.items()):
        w = orc.normal_f32(900 + i, n * m, 0.02)
        tensors.append((f"model.layers.0.{nm}.weight", (n, m), 3, orc.quantize_q4_0(w).tobytes()))
    path = _write(tmp_path, hf.write([("architecture", "llama")], tensors))
    lib = _lib.load()
    xs = {2048: orc.normal_f32(11, 2048, 1.0), 5632: orc.normal_f32(12, 5632, 1.0)}
    with hk.HypnoModel.open(path) as model:
        dx = {k: torch.from_numpy(v).cuda() for k, v in xs.items()}
        ys, descs = [], (_lib.GemvDesc * len(shapes))()
        for i, (nm, (n, m)) in enumerate(shapes.items()):
            ptr, nbytes, dt = model.device_tensor(f"model.layers.0.{nm}.weight")
            assert dt == hk.DType.Q4_0 and nbytes == n * m // 32 * 18
            y = torch.empty(n, device="cuda")
            ys.append(y)
            descs[i].y, descs[i].w_q, descs[i].w_len = y.data_ptr(), ptr, nbytes
            descs[i].x, descs[i].bias, descs[i].n, descs[i].m = dx[m].data_ptr(), None, n, m
        plan = ctypes.c_void_p()
        _lib.check(lib.hypno_hip_q4_0_gemv_plan_create(descs, len(shapes), ctypes.byref(plan)),
                   "plan_create")
        try:
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            _lib.check(lib.hypno_hip_q4_0_gemv_plan_run(plan, st), "plan_run")
            torch.cuda.synchronize()
        finally:
            lib.hypno_hip_q4_0_gemv_plan_destroy(plan)
        for (nm, (n, m)), y in zip(shapes.items(), ys):
            wq = np.frombuffer(bytes(model.get_tensor_data(f"model.layers.0.{nm}.weight")[0]),
                               np.uint8)
            ref = orc.matmul_q4_0(wq, xs[m], None, n, m)
            got = y.cpu().numpy()
            err = np.abs(got - ref).max() / np.abs(ref).max()
            assert err <= 1e-4, (nm, err)
