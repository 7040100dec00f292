"""GGUF v3 reader (host code, no GPU): the reference's own tests of src/gguf.rs
(:655-759) restated through the C ABI, plus round trips of files written by
tests/gguf_writer.py, the metadata key handling of populate_metadata
(src/gguf.rs:517-637) and the error paths of GGUFReader::open."""
import os

import numpy as np
import pytest

import laguna_hip as lh
from gguf_writer import (ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64, f32_bytes, gguf_bytes,
                         write_gguf)

Q4_K, Q8_0, BF16, F32T, F16 = 12, 8, 30, 0, 1


def _open(tmp_path, fields, tensors, name="m.gguf", **kw):
    p = tmp_path / name
    write_gguf(str(p), fields, tensors, **kw)
    return lh.GGUFReader(str(p))


# ---- src/gguf.rs tests (:655-759) ------------------------------------------------------

def test_block_elements():
    assert lh.gguf_type_info(0)[1] == 1
    assert lh.gguf_type_info(8)[1] == 32
    assert lh.gguf_type_info(12)[1] == 256


def test_supported_types():
    for t in (F32T, F16, BF16, Q8_0, Q4_K):
        assert lh.gguf_type_info(t)[2]
    assert not lh.gguf_type_info(4)[2]  # Q5_0


def test_block_sizes():
    assert [lh.gguf_type_info(t)[0] for t in (F32T, F16, BF16, Q8_0, Q4_K)] == [4, 2, 2, 34, 144]


@pytest.mark.parametrize("shape,dtype,elems,nbytes", [
    ([100, 200], BF16, 20000, 40000),        # test_tensor_n_bytes_bf16
    ([100, 200], F32T, 20000, 80000),        # test_tensor_n_bytes_f32
    ([1024], Q8_0, 1024, 1088),              # test_tensor_n_bytes_q8_0
    ([256, 10, 3], Q4_K, 7680, 30 * 144),    # test_tensor_n_bytes_q4_k_3d
])
def test_tensor_n_bytes(tmp_path, shape, dtype, elems, nbytes):
    rd = _open(tmp_path, [], [("test", shape, dtype, bytes(nbytes))])
    t = rd.tensors[0]
    assert (t.n_elements(), t.n_bytes()) == (elems, nbytes)


def test_tensor_type_from_u32():
    # ids 0, 8, 12, 30 are F32, Q8_0, Q4_K, BF16; 10 and 11 decode as Q2_K and Q3_K;
    # ids from_u32 has no arm for are rejected (the reference panics)
    assert lh.gguf_type_info(10)[:2] == lh.gguf_type_info(6)[:2]
    assert lh.gguf_type_info(11)[:2] == lh.gguf_type_info(7)[:2]
    for bad in (31, 32, 33, 36, 37, 38, 42, -1):
        with pytest.raises(lh.LagunaError) as e:
            lh.gguf_type_info(bad)
        assert e.value.status == lh.EINVAL


def test_value_as_string_and_u64(tmp_path):
    # test_value_as_string / test_value_as_u64: as_u64 of U32 and U64, no string of U32,
    # no integer of a string
    rd = _open(tmp_path, [("s", STR, "hello"), ("a", U32, 42), ("b", U64, 100)], [])
    assert rd.field("s") == "hello" and rd.field("a") == 42 and rd.field("b") == 100
    L, h = lh.lib(), rd._h
    out = lh.ctypes.c_uint64()
    assert L.lg_gguf_get_u64(h, rd.find_field("s"), lh.WHOLE, lh.ctypes.byref(out)) == lh.EINVAL
    sp = lh.ctypes.c_char_p()
    assert L.lg_gguf_get_str(h, rd.find_field("a"), lh.WHOLE, lh.ctypes.byref(sp), None) == lh.EINVAL
    assert rd.find_field("absent") is None
    assert L.lg_gguf_find_field(h, b"absent", lh.ctypes.byref(out)) == lh.ENOTFOUND
    with pytest.raises(lh.LagunaError):
        rd.field("absent")


# ---- round trips ------------------------------------------------------------------------

ALL_TYPES = [("u8", U8, 200), ("i8", I8, -5), ("u16", U16, 60000), ("i16", I16, -30000), ("u32", U32, 4000000000),
             ("i32", I32, -7), ("f32", F32, 1.5), ("bool", BOOL, True), ("str", STR, "dflash"),
             ("u64", U64, 2**63 + 5), ("i64", I64, -(2**40)), ("f64", F64, 0.1),
             ("arr", ARR, (I32, [3, -1, 7])), ("sarr", ARR, (STR, ["a", "bc"])), ("empty", ARR, (U32, []))]


def test_every_value_type_round_trips(tmp_path):
    rd = _open(tmp_path, ALL_TYPES, [])
    assert rd.version == 3 and rd.field_count == len(ALL_TYPES) and rd.tensor_count == 0
    got = dict(rd.metadata.raw_fields)
    assert [k for k, _ in rd.metadata.raw_fields] == [k for k, _, _ in ALL_TYPES]
    for key, t, v in ALL_TYPES:
        if t == ARR:
            assert got[key] == list(v[1])
        elif t == F32:
            assert got[key] == np.float32(v)
        else:
            assert got[key] == v, key


def test_as_u64_as_f32_as_bool_conversions(tmp_path):
    # GGUFValue::as_u64 takes U32/U64/I32/I64 (negatives wrap), not U8/U16/floats;
    # as_f32 takes floats and those integers; as_bool takes bools, those integers and floats
    rd = _open(tmp_path, ALL_TYPES, [])
    L, h, c = lh.lib(), rd._h, lh.ctypes
    u, f, b = c.c_uint64(), c.c_float(), c.c_int()
    assert L.lg_gguf_get_u64(h, rd.find_field("i32"), lh.WHOLE, c.byref(u)) == 0 and u.value == 2**64 - 7
    assert L.lg_gguf_get_u64(h, rd.find_field("i64"), lh.WHOLE, c.byref(u)) == 0 and u.value == 2**64 - 2**40
    for k in ("u8", "u16", "f32", "bool", "str", "arr"):
        assert L.lg_gguf_get_u64(h, rd.find_field(k), lh.WHOLE, c.byref(u)) == lh.EINVAL, k
    assert L.lg_gguf_get_f32(h, rd.find_field("u32"), lh.WHOLE, c.byref(f)) == 0 and f.value == np.float32(4e9)
    assert L.lg_gguf_get_f32(h, rd.find_field("i32"), lh.WHOLE, c.byref(f)) == 0 and f.value == -7.0
    assert L.lg_gguf_get_f32(h, rd.find_field("f64"), lh.WHOLE, c.byref(f)) == 0 and f.value == np.float32(0.1)
    assert L.lg_gguf_get_f32(h, rd.find_field("u8"), lh.WHOLE, c.byref(f)) == lh.EINVAL
    assert L.lg_gguf_get_bool(h, rd.find_field("f32"), lh.WHOLE, c.byref(b)) == 0 and b.value == 1
    assert L.lg_gguf_get_bool(h, rd.find_field("u16"), lh.WHOLE, c.byref(b)) == lh.EINVAL
    # array elements
    assert L.lg_gguf_get_u64(h, rd.find_field("arr"), 2, c.byref(u)) == 0 and u.value == 7
    assert L.lg_gguf_get_u64(h, rd.find_field("arr"), 3, c.byref(u)) == lh.EINVAL
    assert L.lg_gguf_get_u64(h, rd.find_field("u32"), 0, c.byref(u)) == lh.EINVAL  # not an array


@pytest.mark.parametrize("alignment", [None, 64, 1, 256])
def test_tensor_data_round_trips_at_any_alignment(tmp_path, alignment):
    rng = np.random.default_rng(7)
    tensors = [("a", [33], F32T, rng.integers(0, 256, 132, np.uint8).tobytes()),
               ("blk.0.ffn_down.weight", [512, 3], Q4_K, rng.integers(0, 256, 6 * 144, np.uint8).tobytes()),
               ("c", [64, 2], Q8_0, rng.integers(0, 256, 4 * 34, np.uint8).tobytes())]
    fields = [("general.architecture", STR, "dflash")]
    a = 32 if alignment is None else alignment
    if alignment is not None:
        fields.append(("general.alignment", U32, alignment))
    p = tmp_path / "t.gguf"
    data_start, offsets = write_gguf(str(p), fields, tensors, alignment=a)
    rd = lh.GGUFReader(str(p))
    assert rd.tensor_data_offset == data_start and data_start % a == 0
    for (name, shape, dt, raw), off, t in zip(tensors, offsets, rd.tensors):
        assert (t.name, t.shape, t.dtype, t.data_offset) == (name, shape, dt, off)
        assert rd.read_tensor_data(t).tobytes() == raw
    assert rd.tensor_by_name("c") is rd.tensors[2]
    assert rd.tensor_by_name("nope") is None
    assert rd.tensors_with_dtype(Q4_K) == [rd.tensors[1]]


def test_first_tensor_of_a_name_wins(tmp_path):
    rd = _open(tmp_path, [], [("x", [4], F32T, f32_bytes([1, 2, 3, 4])), ("x", [4], F32T, f32_bytes([5, 6, 7, 8]))])
    assert np.array_equal(rd.read_tensor_data(rd.tensor_by_name("x")).view(np.float32), [1, 2, 3, 4])


# ---- populate_metadata -------------------------------------------------------------------

def test_model_keys_and_aliases(tmp_path):
    rd = _open(tmp_path, [
        ("general.architecture", STR, "dflash"), ("general.name", STR, "draft"),
        ("dflash.block_count", U32, 6), ("laguna.embedding_length", U64, 4096), ("feed_forward_length", I32, 14336),
        ("dflash.attention.head_count", U32, 32), ("dflash.attention.head_count_kv", U32, 8),
        ("dflash.attention.key_length", U32, 128), ("dflash.attention.layer_norm_rms_epsilon", F32, 1e-5),
        ("dflash.rope.freq_base", U32, 500000), ("rope.dimension_count", U32, 128),
        ("dflash.target_layers", ARR, (I32, [2, 18, 33])), ("vocab_size", U32, 100352),
        ("dflash.decoder_arch", STR, "qwen3"), ("expert_weights_norm", U32, 1), ("unrelated.key", U32, 3)], [])
    m = rd.metadata
    assert (m.architecture, m.general_name, m.block_count, m.embedding_length, m.feed_forward_length) == \
        ("dflash", "draft", 6, 4096, 14336)
    assert (m.attention_head_count, m.attention_head_count_kv, m.attention_key_length) == (32, 8, 128)
    assert m.attention_layer_norm_rms_epsilon == np.float32(1e-5)
    assert m.rope_freq_base == 500000.0 and m.rope_dimension_count == 128  # as_f32 of a u32
    assert m.target_layers == [2, 18, 33] and m.vocab_size == 100352 and m.decoder_arch == "qwen3"
    assert m.expert_weights_norm is True and m.context_length is None and m.alignment is None
    assert rd.layer_count() == 6 and rd.embedding_length() == 4096


def test_head_count_arrays(tmp_path):
    # an array head count gives its first entry; an array kv count its second (only
    # when it has one; a one-element array leaves the field as it was)
    rd = _open(tmp_path, [("attention.head_count", ARR, (U32, [40, 48])),
                          ("attention.head_count_kv", ARR, (U32, [4, 8, 16]))], [])
    assert rd.metadata.attention_head_count == 40 and rd.metadata.attention_head_count_kv == 8
    rd = _open(tmp_path, [("attention.head_count_kv", U32, 2), ("attention.head_count_kv", ARR, (U32, [4]))], [],
               name="b.gguf")
    assert rd.metadata.attention_head_count_kv == 2


def test_later_key_overwrites_and_bad_type_clears(tmp_path):
    rd = _open(tmp_path, [("block_count", U32, 4), ("dflash.block_count", U32, 6), ("embedding_length", U32, 8),
                          ("embedding_length", STR, "x")], [])
    assert rd.metadata.block_count == 6 and rd.metadata.embedding_length is None


def test_target_layers_skip_non_integers_and_general_rope_quirk(tmp_path):
    rd = _open(tmp_path, [("target_layers", ARR, (U8, [1, 2])), ("general.x.rope_dimension_count", ARR, (U64, [64, 1]))],
               [])
    assert rd.metadata.target_layers == []  # u8 entries have no as_u64
    assert rd.metadata.rope_dimension_count == 64


# ---- GGUFReader::open errors ---------------------------------------------------------------

def _status(tmp_path, blob):
    p = tmp_path / "bad.gguf"
    p.write_bytes(blob)
    with pytest.raises(lh.LagunaError) as e:
        lh.GGUFReader(str(p))
    return e.value.status, str(e.value)


def test_open_errors(tmp_path):
    good, data_start, _ = gguf_bytes([("k", U32, 1)], [("t", [8], F32T, f32_bytes(np.arange(8)))])
    st, msg = _status(tmp_path, b"GGML" + good[4:])
    assert st == lh.EIO and "not a GGUF file" in msg
    st, msg = _status(tmp_path, gguf_bytes([], [], version=2)[0])
    assert st == lh.EIO and "v2" in msg
    hdr_len = gguf_bytes([("k", U32, 1)], [("t", [8], F32T, b"")], alignment=1)[1]  # header without padding
    for cut in (3, 10, 30, hdr_len - 5):  # inside the magic, the counts, the field, the tensor info
        assert _status(tmp_path, good[:cut])[0] == lh.EIO, cut
    st, msg = _status(tmp_path, gguf_bytes([], [("t", [8], 31, bytes(32))])[0])
    assert st == lh.EIO and "unknown type" in msg
    with pytest.raises(lh.LagunaError) as e:
        lh.GGUFReader(str(tmp_path / "missing.gguf"))
    assert e.value.status == lh.EIO


def test_unknown_value_type_is_an_error(tmp_path):
    blob = bytearray(gguf_bytes([("k", U32, 1)], [])[0])
    # the field's type id sits after magic, version, counts and the key
    pos = 4 + 4 + 8 + 8 + 8 + 1
    blob[pos:pos + 4] = (13).to_bytes(4, "little")
    st, msg = _status(tmp_path, bytes(blob))
    assert st == lh.EIO and "type 13" in msg


def test_tensor_past_end_of_file(tmp_path):
    blob, _, _ = gguf_bytes([], [("t", [64], F32T, f32_bytes(np.arange(64)))])
    p = tmp_path / "short.gguf"
    p.write_bytes(blob[:-8])
    rd = lh.GGUFReader(str(p))
    with pytest.raises(lh.LagunaError) as e:
        rd.read_tensor_data(rd.tensors[0])
    assert e.value.status == lh.EIO
    buf = np.empty(8, np.uint8)
    assert lh.lib().lg_gguf_read_tensor(rd._h, 0, buf.ctypes.data, buf.size) != 0  # destination too small too


def test_closed_reader_releases_the_file(tmp_path):
    rd = _open(tmp_path, [], [("t", [4], F32T, f32_bytes([1, 2, 3, 4]))])
    fd_count = len(os.listdir("/proc/self/fd"))
    rd.close()
    assert len(os.listdir("/proc/self/fd")) == fd_count - 1
