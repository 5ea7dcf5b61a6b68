"""Safetensors reading and writing in the library (host-only, no GPU), against
the reference's own fixtures: hex dumps of files written by the `safetensors`
Python package (crates/midman-checkpoint/tests/fixtures/*.hex, copied as data
into tests/golden/safetensors/), and the reference's unit tests of the format
(crates/midman-checkpoint/src/safetensors.rs:462-760,
tests/reference_files.rs:36-148)."""
import math
import os
import struct

import numpy as np
import pytest

import midman_hip as mh

HERE = os.path.dirname(os.path.abspath(__file__))


def fixture(name):
    with open(os.path.join(HERE, "golden", "safetensors", name + ".hex")) as f:
        return bytes.fromhex("".join(f.read().split()))


def bits(values):
    return np.asarray(values, np.float32).view(np.uint32).tolist()


BASIC = [  # reference_files.rs:36-48, in file order
    ("b", [3], [0.1, 0.2, 0.3]),
    ("empty", [0], []),
    ("scalar", [], [7.0]),
    ("special", [6], [math.nan, math.inf, -math.inf, -0.0, np.finfo(np.float32).tiny, 1e-45]),
    ("w", [2, 3], [1.5, -2.0, 0.0, 3.25, 1e-30, 1e30]),
]


def raw_file(header: str, data: bytes) -> bytes:
    h = header.encode("utf-8")
    return struct.pack("<Q", len(h)) + h + data


def floats(vals):
    return np.asarray(vals, np.float32).tobytes()


def test_reads_the_reference_file_with_every_shape_and_special_value():
    f = mh.TensorFile.from_bytes(fixture("basic"))
    assert f.metadata() == {"format": "pt"}
    got = f.tensors()
    assert len(got) == len(BASIC)
    for (name, shape, vals), (en, es, ev) in zip(got, BASIC):
        assert name == en and shape == es
        assert bits(vals) == bits(ev), name


def test_writes_exactly_the_bytes_the_reference_writes():
    f = mh.TensorFile()
    for name, shape, vals in BASIC:
        f.push(name, shape, vals)
    f.set_metadata("format", "pt")
    assert f.to_bytes() == fixture("basic")


def test_unicode_quotes_tabs_newlines_match_byte_for_byte():
    data = fixture("unicode_names")
    f = mh.TensorFile.from_bytes(data)
    t = {n: v.tolist() for n, _, v in f.tensors()}
    assert t["layer.0.é日本"] == [1.0, 2.0]
    assert t['quote"back\\slash\ttab'] == [3.0]
    assert f.metadata() == {"note": 'café "quoted" 日本\nline'}
    again = mh.TensorFile()
    again.push("layer.0.é日本", [2], [1.0, 2.0])
    again.push('quote"back\\slash\ttab', [1], [3.0])
    again.set_metadata("note", 'café "quoted" 日本\nline')
    assert again.to_bytes() == data


def test_the_empty_file_matches_the_reference_both_ways():
    data = fixture("empty")
    f = mh.TensorFile.from_bytes(data)
    assert f.tensors() == [] and f.metadata() == {}
    assert mh.TensorFile().to_bytes() == data
    assert data == raw_file("{}      ", b"")


def test_several_metadata_entries_are_rewritten_sorted():
    f = mh.TensorFile.from_bytes(fixture("multi_metadata"))
    assert list(f.metadata().items()) == [("alpha", "1"), ("beta", "2"), ("gamma", "3")]
    assert {n: v.tolist() for n, _, v in f.tensors()}["x"] == [1.0]
    text = f.to_bytes().decode("utf-8", "replace")
    assert text.find('"alpha"') < text.find('"beta"') < text.find('"gamma"')
    assert mh.TensorFile.from_bytes(f.to_bytes()).metadata() == f.metadata()


def test_a_reference_file_with_another_dtype_is_rejected_by_name():
    with pytest.raises(mh.MidmanError) as e:
        mh.TensorFile.from_bytes(fixture("mixed_dtypes"))
    assert "`h`" in e.value.message and "F16" in e.value.message


def test_no_prefix_of_a_file_is_accepted_and_trailing_bytes_are_rejected():
    data = fixture("basic")
    for n in range(len(data)):
        with pytest.raises(mh.MidmanError):
            mh.TensorFile.from_bytes(data[:n])
    mh.TensorFile.from_bytes(data).close()
    with pytest.raises(mh.MidmanError):
        mh.TensorFile.from_bytes(data + b"\0")


def test_flipping_any_single_bit_never_crashes():
    for data in (fixture("basic"), fixture("unicode_names")):
        for pos in range(len(data)):
            for bit in range(8):
                c = bytearray(data)
                c[pos] ^= 1 << bit
                try:
                    mh.TensorFile.from_bytes(bytes(c)).close()
                except mh.MidmanError:
                    pass


def test_round_trips_every_bit_including_nan_payloads_and_signed_zero():
    tricky = np.array([0x7fc01234, 0x7f800000, 0x80000000, 0x00000001, 0xff800000, 0x3f800000],
                      np.uint32).view(np.float32)
    f = mh.TensorFile()
    f.push("t", [6], tricky)
    back = mh.TensorFile.from_bytes(f.to_bytes()).tensors()
    assert back[0][2].view(np.uint32).tolist() == tricky.view(np.uint32).tolist()


def test_writes_sorted_by_name_with_a_header_padded_to_eight_bytes():
    f = mh.TensorFile()
    f.push("w", [2, 3], [1.5, -2.0, 0.0, 3.25, 1e-30, 1e30])
    f.push("b", [3], [0.1, 0.2, 0.3])
    f.set_metadata("format", "test")
    data = f.to_bytes()
    hl = struct.unpack("<Q", data[:8])[0]
    assert hl % 8 == 0
    assert data[8:8 + hl].decode().rstrip() == (
        '{"__metadata__":{"format":"test"},'
        '"b":{"dtype":"F32","shape":[3],"data_offsets":[0,12]},'
        '"w":{"dtype":"F32","shape":[2,3],"data_offsets":[12,36]}}')
    assert len(data) == 8 + hl + 36
    for n in range(1, 25):
        g = mh.TensorFile()
        g.push("a" * n, [1], [1.0])
        d = g.to_bytes()
        hl = struct.unpack("<Q", d[:8])[0]
        h = d[8:8 + hl].decode()
        assert hl % 8 == 0 and len(h) - len(h.rstrip()) < 8


def test_reading_orders_by_data_position_and_accepts_trailing_whitespace():
    h = ('{"a":{"dtype":"F32","shape":[1],"data_offsets":[4,8]},'
         '"z":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')
    t = mh.TensorFile.from_bytes(raw_file(h, floats([1.0, 2.0]))).tensors()
    assert [n for n, _, _ in t] == ["z", "a"] and t[1][2].tolist() == [2.0]
    h2 = '{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}} \n\t  '
    assert mh.TensorFile.from_bytes(raw_file(h2, floats([9.0]))).tensors()[0][2].tolist() == [9.0]


def test_push_rejects_bad_tensors():
    f = mh.TensorFile()
    with pytest.raises(mh.ShapeError):
        f.push("a", [2, 2], [1.0, 2.0, 3.0])
    with pytest.raises(mh.ShapeError):
        f.push("a", [2 ** 64 - 1, 2], [])
    with pytest.raises(mh.ArgumentError):
        f.push("__metadata__", [1], [1.0])
    f.push("a", [1], [1.0])
    with pytest.raises(mh.ArgumentError):
        f.push("a", [1], [2.0])
    assert len(f.tensors()) == 1


def one(dtype, shape, begin, end):
    return f'{{"a":{{"dtype":"{dtype}","shape":{shape},"data_offsets":[{begin},{end}]}}}}'


def test_rejects_malformed_files():
    four = floats([1.0])
    good = one("F32", "[1]", 0, 4)
    mh.TensorFile.from_bytes(raw_file(good, four)).close()
    cases = {
        "short prefix": bytes([2, 0, 0, 0, 0, 0, 0]),
        "header length of u64::MAX": struct.pack("<Q", 2 ** 64 - 1) + b"{}",
        "header past the end": struct.pack("<Q", 50) + b"{}",
        "header over the limit": struct.pack("<Q", 100000001) + b"{}",
        "not starting with {": raw_file(" {}", b""),
        "not UTF-8": struct.pack("<Q", 3) + b"{\xff}",
        "not an object": raw_file("[]", b""),
        "unsupported dtype": raw_file(one("F16", "[1]", 0, 2), b"\0\0"),
        "lowercase dtype": raw_file(one("f32", "[1]", 0, 4), four),
        "shape against range": raw_file(one("F32", "[2]", 0, 4), four),
        "end before begin": raw_file(one("F32", "[1]", 4, 0), four),
        "range past the data": raw_file(one("F32", "[1]", 0, 4), b"\0\0"),
        "trailing bytes": raw_file(good, floats([1.0, 2.0])),
        "gap before the first tensor": raw_file(one("F32", "[1]", 4, 8), floats([1.0, 2.0])),
        "shape overflow": raw_file(one("F32", "[4294967296,4294967296,4294967296]", 0, 4), four),
        "dimension too large": raw_file(one("F32", "[18446744073709551616]", 0, 4), four),
        "negative dimension": raw_file(one("F32", "[-1]", 0, 4), four),
        "unknown field": raw_file('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4],"extra":1}}',
                                  four),
        "missing field": raw_file('{"a":{"dtype":"F32","shape":[1]}}', four),
        "entry not an object": raw_file('{"a":1}', four),
        "three offsets": raw_file('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4,8]}}', four),
        "metadata not strings": raw_file('{"__metadata__":{"k":1}}', b""),
        "metadata not an object": raw_file('{"__metadata__":["k"]}', b""),
        "duplicate names": raw_file('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},'
                                    '"a":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}',
                                    floats([1.0, 2.0])),
        "fraction": raw_file(one("F32", "[1.0]", 0, 4), four),
        "leading zero": raw_file(one("F32", "[01]", 0, 4), four),
        "boolean": raw_file('{"a":true}', b""),
        "unpaired surrogate": raw_file('{"\\ud800":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}',
                                       four),
        "nesting too deep": raw_file('{"__metadata__":' + "[" * 9 + "]" * 9 + "}", b""),
    }
    for what, data in cases.items():
        with pytest.raises(mh.MidmanError):
            mh.TensorFile.from_bytes(data)
            pytest.fail(f"should reject: {what}")


def test_limit_overlap_and_lying_sizes_are_refused_for_their_reason():
    with pytest.raises(mh.MidmanError) as e:
        mh.TensorFile.from_bytes(struct.pack("<Q", 100000001) + b"{}")
    assert "limit" in e.value.message
    with pytest.raises(mh.MidmanError) as e:
        mh.TensorFile.from_bytes(struct.pack("<Q", 100000000) + b"{}")
    assert "limit" not in e.value.message
    h = ('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
         '"b":{"dtype":"F32","shape":[2],"data_offsets":[4,12]}}')
    with pytest.raises(mh.MidmanError) as e:
        mh.TensorFile.from_bytes(raw_file(h, floats([1.0, 2.0, 3.0])))
    assert "no gap or overlap" in e.value.message
    with pytest.raises(mh.MidmanError) as e:
        mh.TensorFile.from_bytes(raw_file(one("F32", "[1000000000]", 0, 4000000000), floats([1.0])))
    assert "cover" in e.value.message
    with pytest.raises(mh.MidmanError) as e:
        mh.TensorFile.from_bytes(raw_file(one("BF16", "[1]", 0, 2), b"\0\0"))
    assert "safetensors file" in e.value.message and "`a`" in e.value.message
    assert "BF16" in e.value.message


def test_escapes_match_the_serde_json_rules():
    # json.rs:51-67: quote, backslash, \b \f \n \r \t, other controls as \u00XX,
    # everything else (including non-ASCII and '/') verbatim.
    f = mh.TensorFile()
    name = 'a"b\\c\bd\fe\nf\rg\th\x01i\x1fj/ké'
    f.push(name, [1], [1.0])
    data = f.to_bytes()
    hl = struct.unpack("<Q", data[:8])[0]
    want = '"a\\"b\\\\c\\bd\\fe\\nf\\rg\\th\\u0001i\\u001fj/ké"'
    assert want in data[8:8 + hl].decode("utf-8")
    assert mh.TensorFile.from_bytes(data).tensors()[0][0] == name


def test_parameter_names_follow_the_reference():
    names = mh.parameter_names([12, 16, 2, 2, 1, 32, 16, 1e4, 1e-5, 0])
    assert names[0] == "embed_tokens.weight" and names[-1] == "lm_head.weight"
    assert names[1:10] == ["blocks.0.attn_norm.weight", "blocks.0.attn.q_proj.weight",
                           "blocks.0.attn.k_proj.weight", "blocks.0.attn.v_proj.weight",
                           "blocks.0.attn.o_proj.weight", "blocks.0.mlp_norm.weight",
                           "blocks.0.mlp.gate_proj.weight", "blocks.0.mlp.up_proj.weight",
                           "blocks.0.mlp.down_proj.weight"]
    assert len(set(names)) == len(names) == 1 + 9 * 2 + 2
