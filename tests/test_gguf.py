"""GGUF reader: header, metadata, tensor directory and tensor bytes, checked against files this
test writes in the published GGUF v3 layout (the one the reference's probe/phase63_gguf_header.py
reads), plus malformed files that must be rejected. No GGUF model ships with the reference, so
the fixtures are synthetic.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import _oracle as O

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
PACK = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def gval(t: int, v) -> bytes:
    if t == STR:
        return gstr(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(gval(et, x) for x in items)
    return struct.pack(PACK[t], v)


def write_gguf(path, kv, tensors, alignment=32, version=3):
    """kv: [(key, type, value)]; tensors: [(name, ne tuple, ggml_type, bytes)]."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kv))
    for k, t, v in kv:
        head += gstr(k) + struct.pack("<I", t) + gval(t, v)
    offs, data = [], b""
    for _, _, _, raw in tensors:
        data += b"\0" * (-len(data) % alignment)
        offs.append(len(data))
        data += raw
    for (name, ne, gt, _), off in zip(tensors, offs):
        head += gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", gt, off)
    head += b"\0" * (-len(head) % alignment)
    path.write_bytes(head + data)
    return len(head), offs


def q8_tensor(N, K, seed):
    q = ((O.uniform(N * K, seed, 0.0, 1.0) * 255).astype(np.int32) - 127).astype(np.int8).reshape(N, K)
    d = O.f16_bits(O.uniform(N * K // 32, seed + 1, 1e-3, 1e-2)).reshape(N, K // 32)
    return O.q8_0_pack(q, d)


@pytest.fixture
def model(tmp_path):
    W = q8_tensor(48, 256, 3)
    H = O.f16_bits(O.normal(32, 4, 0, 1))
    F = O.normal(10, 5, 0, 1)
    kv = [("general.architecture", STR, "llama"), ("general.name", STR, "synthetic"),
          ("llama.embedding_length", U32, 256), ("llama.block_count", U32, 1),
          ("llama.attention.layer_norm_rms_epsilon", F32, 1e-6), ("general.file_type", U32, 7),
          ("tokenizer.ggml.tokens", ARR, (STR, ["<s>", "</s>", "a"])), ("some.i64", I64, -5),
          ("some.flags", ARR, (U8, [1, 2, 3])), ("some.bool", BOOL, True), ("some.f64", F64, 0.25)]
    tensors = [("blk.0.ffn_up.weight", (256, 48), 8, W.tobytes()), ("blk.0.attn_norm.weight", (32,), 1, H.tobytes()),
               ("output_norm", (10,), 0, F.tobytes())]
    p = tmp_path / "m.gguf"
    head, offs = write_gguf(p, kv, tensors)
    return p, W, H, F, head, offs


def test_directory_and_metadata(uk, model):
    p, W, H, F, head, offs = model
    with uk.Gguf(p) as g:
        assert len(g) == 3
        t = g.tensor("blk.0.ffn_up.weight")
        assert (t.index, t.type_name, t.ne, t.nbytes) == (0, "q8_0", (256, 48), W.nbytes)
        assert t.offset == head + offs[0] and t.offset % 32 == 0
        assert g.tensor(1).name == "blk.0.attn_norm.weight" and g.tensor(1).nbytes == 64
        assert g.tensor("output_norm").nbytes == 40
        assert g.metadata("general.architecture") == "llama"
        assert g.metadata("llama.embedding_length") == "256"
        assert g.metadata("some.i64") == "-5" and g.metadata("some.bool") == "true"
        assert g.metadata("tokenizer.ggml.tokens") == "[3 x type 8]"
        assert g.metadata("absent") is None
        with pytest.raises(KeyError):
            g.tensor("absent")


def test_tensor_bytes_and_q8_desc(uk, model):
    p, W, H, F, *_ = model
    with uk.Gguf(p) as g:
        assert np.array_equal(g.read("blk.0.ffn_up.weight"), W)
        assert np.array_equal(g.read(1).view(np.uint16), H)
        assert np.array_equal(g.read(2).view(np.float32), F)
        d = g.q8_0_desc("blk.0.ffn_up.weight", 16)
        assert uk.op_signature(d) == "gemm:q8_0:16x48x256:TN"
        assert uk.workload_of(d)["weight_bytes"] == W.nbytes
        with pytest.raises(uk.UnikernError):
            g.q8_0_desc("output_norm", 1)  # not q8_0


def test_alignment_metadata_is_honoured(uk, tmp_path):
    W = q8_tensor(16, 64, 9)
    p = tmp_path / "a.gguf"
    head, offs = write_gguf(p, [("general.alignment", U32, 256)],
                            [("x", (3,), 0, O.normal(3, 1, 0, 1).tobytes()), ("w", (64, 16), 8, W.tobytes())],
                            alignment=256)
    with uk.Gguf(p) as g:
        t = g.tensor("w")
        assert t.offset == head + offs[1] and t.offset % 256 == 0
        assert np.array_equal(g.read("w"), W)


@pytest.mark.parametrize("mutate,needle", [
    (lambda b: b"XXXX" + b[4:], "bad magic"),
    (lambda b: b[:4] + struct.pack("<I", 7) + b[8:], "version"),
    (lambda b: b[:40], "end of file"),
])
def test_malformed_files_are_rejected(uk, model, tmp_path, mutate, needle):
    p = model[0]
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(mutate(p.read_bytes()))
    with pytest.raises(uk.UnikernError) as e:
        uk.Gguf(bad)
    assert needle in str(e.value)


def test_tensor_past_end_and_too_many_dims(uk, tmp_path):
    p = tmp_path / "t.gguf"
    write_gguf(p, [], [("w", (64, 16), 8, q8_tensor(16, 64, 1).tobytes())])
    raw = p.read_bytes()
    (tmp_path / "short.gguf").write_bytes(raw[:-100])
    with pytest.raises(uk.UnikernError) as e:
        uk.Gguf(tmp_path / "short.gguf")
    assert "past the end" in str(e.value)
    q = tmp_path / "dims.gguf"
    write_gguf(q, [], [("w", (2, 2, 2, 2, 2), 0, b"\0" * 128)])
    with pytest.raises(uk.UnikernError) as e:
        uk.Gguf(q)
    assert "dims" in str(e.value)


@pytest.mark.gpu
def test_q8_0_gemm_from_gguf_tensor(gpu, tmp_path):
    # A Llama-7B-shaped projection (K = 4096, N = 4096) read from a GGUF file straight into HBM
    # and multiplied by the Q8_0 kernel; checked against the binary64 oracle.
    N, K, M = 4096, 4096, 8
    W = q8_tensor(N, K, 20261201 + 41)
    p = tmp_path / "proj.gguf"
    write_gguf(p, [("general.architecture", STR, "llama")], [("blk.0.attn_q.weight", (K, N), 8, W.tobytes())])
    Xh = O.f16_bits(O.normal(M * K, 20261201 + 40, 0.0, 1.0)).reshape(M, K)
    with gpu.Gguf(p) as g:
        wb = g.upload("blk.0.attn_q.weight")
        d = g.q8_0_desc("blk.0.attn_q.weight", M)
    xb = gpu.DeviceBuffer.from_array(Xh)
    yb = gpu.DeviceBuffer(M * N * 4)
    gpu.launch(d, [xb, wb], yb)
    y = yb.download(np.float32, (M, N)).astype(np.float64)
    r = O.q8_0_gemm(Xh, W, N)
    assert np.linalg.norm(y - r) / np.linalg.norm(r) <= 1e-5
