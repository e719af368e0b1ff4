"""The GGUF reader (csrc/host/gguf.cpp via llamd_rs_amd.gguf) against files
whose every byte the test wrote: metadata of every type, tensors of the four
types the path reads, alignment, and each malformed-file rule of the
reference parser (crates/llamd-gguf/src/lib.rs:141-236, 256-278, 293-375).
Host-only: no device is touched."""
import math
import struct

import numpy as np
import pytest

from llamd_rs_amd import gguf_writer as W
from llamd_rs_amd._lib import HipError, lib

try:
    lib()
    HAVE_LIB = True
except Exception:
    HAVE_LIB = False
pytestmark = pytest.mark.skipif(not HAVE_LIB, reason="libllamd_hip.so is not built")


def open_gguf(path):
    from llamd_rs_amd.gguf import Gguf
    return Gguf(path)


def rng_bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


ALL_KVS = [
    ("general.architecture", W.STRING, "qwen3moe"),
    ("a.u8", W.U8, 250), ("a.i8", W.I8, -7), ("a.u16", W.U16, 65000), ("a.i16", W.I16, -30000),
    ("a.u32", W.U32, 4_000_000_000), ("a.i32", W.I32, -2_000_000_000), ("a.f32", W.F32, 1.5e-6),
    ("a.bool", W.BOOL, True), ("a.u64", W.U64, 2**63 + 5), ("a.i64", W.I64, -2**62),
    ("a.f64", W.F64, math.pi), ("a.str", W.STRING, "héllo"),
    ("a.arr_i32", W.ARRAY, (W.I32, [1, -2, 3])),
    ("a.arr_str", W.ARRAY, (W.STRING, ["x", "", "yz"])),
    ("a.arr_empty", W.ARRAY, (W.F32, [])),
]


def test_metadata_of_every_type_round_trips(tmp_path):
    p = tmp_path / "kv.gguf"
    W.write(p, ALL_KVS, [])
    g = open_gguf(p)
    assert g.version == 3 and g.tensors == []
    assert list(g.metadata) == sorted(k for k, _, _ in ALL_KVS)   # BTreeMap order
    for k, t, v in ALL_KVS:
        got = g.get(k)
        if t == W.F32:
            assert got == struct.unpack("<f", struct.pack("<f", v))[0]
        elif t == W.ARRAY:
            assert got == list(v[1])
        else:
            assert got == v, k
    assert g.architecture() == "qwen3moe"
    assert g.data_offset % 32 == 0 and g.alignment == 32


def test_value_accessors_follow_the_reference(tmp_path):
    """Value::as_u64 takes unsigned types and non-negative signed ones;
    Value::as_f32 takes F32, and F64 rounded (lib.rs:55-74)."""
    p = tmp_path / "acc.gguf"
    W.write(p, ALL_KVS + [("a.i32pos", W.I32, 12)], [])
    g = open_gguf(p)
    L = lib()
    import ctypes as C
    u, f = C.c_uint64(), C.c_float()
    ok = lambda k: L.llamd_gguf_get_u64(g._h, k.encode(), C.byref(u)) == 0
    assert ok("a.u8") and u.value == 250
    assert ok("a.i32pos") and u.value == 12
    assert ok("a.u64") and u.value == 2**63 + 5
    assert not ok("a.i8") and not ok("a.f32") and not ok("a.bool") and not ok("a.str")
    assert not ok("no.such.key")
    assert L.llamd_gguf_get_f32(g._h, b"a.f64", C.byref(f)) == 0
    assert f.value == np.float32(math.pi)
    assert L.llamd_gguf_get_f32(g._h, b"a.u32", C.byref(f)) == -1


def test_duplicate_keys_keep_the_last(tmp_path):
    p = tmp_path / "dup.gguf"
    W.write(p, [("k", W.U32, 1), ("j", W.U32, 2), ("k", W.U32, 3)], [])
    g = open_gguf(p)
    assert g.metadata == {"j": 2, "k": 3}


def q6k_bytes(rows, k, seed):
    return rng_bytes(rows * k // 256 * 210, seed)


@pytest.mark.parametrize("alignment", [32, 64, 4096])
def test_tensors_of_every_type_and_their_bytes(tmp_path, alignment):
    f32 = np.arange(12, dtype=np.float32).tobytes()
    f16 = np.arange(8, dtype=np.float16).tobytes()
    q8 = rng_bytes(2 * 64 // 32 * 34, 3)
    q6 = q6k_bytes(4, 512, 4)
    q6e = q6k_bytes(3 * 2, 256, 5)
    tensors = [("t.f32", [3, 4], 0, f32), ("t.f16", [8], 1, f16), ("t.q8", [64, 2], 8, q8),
               ("t.q6", [512, 4], 14, q6), ("t.q6e", [256, 3, 2], 14, q6e)]
    kvs = [("general.alignment", W.U32, alignment)] if alignment != 32 else []
    p = tmp_path / "t.gguf"
    W.write(p, kvs, tensors, alignment=alignment)
    g = open_gguf(p)
    assert g.alignment == alignment and g.data_offset % alignment == 0
    assert [t.name for t in g.tensors] == [t[0] for t in tensors]
    for (name, dims, ty, data), t in zip(tensors, g.tensors):
        assert t.dims == dims and t.ggml_type == ty and t.offset % alignment == 0
        assert bytes(g.tensor_data(t)) == data, name
    assert g.tensor("t.q6e").elems() == 256 * 3 * 2
    assert g.tensor("absent") is None


def refused(tmp_path, data, fragment):
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    with pytest.raises(HipError) as e:
        open_gguf(p)
    assert fragment in str(e.value), str(e.value)


def test_malformed_headers_are_refused(tmp_path):
    good = W.build([("general.architecture", W.STRING, "qwen3")], [("t", [256], 0, bytes(1024))])
    refused(tmp_path, b"GGUX" + good[4:], "magic")
    refused(tmp_path, W.build([], [], version=2), "version 2")
    refused(tmp_path, good[:10], "truncated")
    refused(tmp_path, W.build([], [], n_kv=1 << 40), "exceeds")
    refused(tmp_path, W.build([], [], n_tensors=1 << 40), "exceeds")
    # a string length far past the end
    bad = bytearray(W.build([("k", W.STRING, "v")], []))
    bad[24:32] = struct.pack("<Q", 1 << 50)
    refused(tmp_path, bytes(bad), "truncated")


def test_malformed_values_are_refused(tmp_path):
    refused(tmp_path, W.build([("k", W.ARRAY, (W.ARRAY, []))], []), "nested")
    head = b"GGUF" + struct.pack("<IQQ", 3, 0, 1)
    refused(tmp_path, head + W.gstr("k") + struct.pack("<I", 13) + b"\x01" * 8, "unknown type 13")
    # an array declaring more elements than bytes remain
    arr = bytearray(W.build([("k", W.ARRAY, (W.U8, [1, 2, 3]))], []))
    i = arr.index(struct.pack("<IQ", W.U8, 3))
    arr[i + 4:i + 12] = struct.pack("<Q", 1 << 40)
    refused(tmp_path, bytes(arr), "elements declared")


def test_malformed_tensor_infos_are_refused(tmp_path):
    refused(tmp_path, W.build([], [("t", [1, 1, 1, 1, 256], 0, bytes(1024))]), "at most 4")
    refused(tmp_path, W.build([("general.alignment", W.U32, 48)], [], alignment=48),
            "not a power of two")
    refused(tmp_path, W.build([("general.alignment", W.U32, 0)], [], alignment=32),
            "not a power of two")
    # the header ends short of the next 4096-byte boundary and the file ends
    # with it: the data section would start past the end
    kv = [("general.alignment", W.U32, 4096)]
    end = len(W.build(kv, [], alignment=1))          # no padding
    refused(tmp_path, W.build(kv, [], alignment=4096)[:end], "past the")


def test_tensor_data_checks_type_length_and_extent(tmp_path):
    p = tmp_path / "td.gguf"
    W.write(p, [], [("ok", [256], 14, bytes(210)), ("q4", [32], 2, bytes(18)),
                    ("odd", [100], 14, bytes(210)), ("far", [256], 0, bytes(1024))])
    # move "far" past the end of the file
    data = bytearray(p.read_bytes())
    i = data.index(W.gstr("far"))
    off_at = i + len(W.gstr("far")) + 4 + 8 + 4
    data[off_at:off_at + 8] = struct.pack("<Q", 1 << 30)
    p.write_bytes(bytes(data))
    g = open_gguf(p)
    assert len(g.tensor_data(g.tensor("ok"))) == 210
    with pytest.raises(HipError, match="not implemented yet"):
        g.tensor_data(g.tensor("q4"))
    with pytest.raises(HipError, match="not a multiple"):
        g.tensor_data(g.tensor("odd"))
    with pytest.raises(HipError, match="past the"):
        g.tensor_data(g.tensor("far"))


def test_open_missing_file_fails_cleanly(tmp_path):
    with pytest.raises(HipError, match="cannot open"):
        open_gguf(tmp_path / "nope.gguf")
    (tmp_path / "empty.gguf").write_bytes(b"")
    with pytest.raises(HipError, match="empty"):
        open_gguf(tmp_path / "empty.gguf")


def test_moe_layer_from_a_gguf_file_refuses_bad_shapes(tmp_path):
    """Shape checks happen before any device work (llamd_gguf_moe_create)."""
    from llamd_rs_amd._lib import HipError
    from llamd_rs_amd.gguf import Gguf
    p = tmp_path / "bad.gguf"
    W.write(p, [("general.architecture", W.STRING, "qwen3moe"),
                ("qwen3moe.expert_used_count", W.U32, 2)],
            [("blk.0.ffn_gate_inp.weight", [256, 4], 0, bytes(4096)),
             ("blk.0.ffn_gate_exps.weight", [256, 256, 4], 14, bytes(210 * 256 * 4)),
             ("blk.0.ffn_up_exps.weight", [256, 256, 4], 14, bytes(210 * 256 * 4)),
             ("blk.0.ffn_down_exps.weight", [256, 512, 4], 14, bytes(210 * 512 * 4))])
    with Gguf(p) as g:
        with pytest.raises(HipError, match="disagree"):
            g.moe_layer(0)
        with pytest.raises(HipError, match="lacks"):
            g.moe_layer(1)


def test_tensors_may_share_their_data(tmp_path):
    """Tensor infos are offsets: two tensors may point at the same bytes (the
    writer stores a repeated data object once)."""
    data = rng_bytes(210 * 4, 9)
    p = tmp_path / "shared.gguf"
    W.write(p, [], [("a", [256, 4], 14, data), ("b", [256, 4], 14, data), ("c", [256], 14, data[:210])])
    g = open_gguf(p)
    ta, tb, tc = g.tensors
    assert ta.offset == tb.offset != tc.offset
    assert bytes(g.tensor_data(ta)) == bytes(g.tensor_data(tb)) == data
    assert g.file_size() < g.data_offset + 3 * len(data)
