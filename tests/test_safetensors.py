"""The safetensors reader of the C ABI (ncm_st_*, host code, no GPU) against
the reference's own checks (packages/safetensors/root.zig:320-439, restated
here case by case) and against the oracle's restatement of the parser on
generated headers, valid and broken."""
import json
import random

import pytest

from ncmorph_amd import safetensors as st
from ncmorph_amd._lib import NcmError


def make_file(js: str, data_len: int) -> bytes:
    raw = js.encode()
    return len(raw).to_bytes(8, "little") + raw + bytes(data_len)


def c_parse(data: bytes, file_size=None):
    """("ok", header_len, data_len, tensors) or ("err", name) from the C ABI."""
    try:
        f = st.SafetensorsFile(data=data, file_size=file_size)
    except NcmError as e:
        return ("err", e.detail)
    hl, dl, _ = f.summary()
    ts = [(t.name, t.dtype, list(t.shape), t.data_begin, t.data_end) for t in f.tensors()]
    f.close()
    return ("ok", hl, dl, ts)


def o_parse(oracle, data: bytes, file_size=None):
    try:
        hl, dl, ts = oracle.st_parse_header(data, len(data) if file_size is None else file_size)
    except oracle.StError as e:
        return ("err", str(e))
    names = [n for n, _ in oracle.ST_DTYPES]
    return ("ok", hl, dl, [(n, names[d], list(s), b, e) for n, d, s, b, e in ts])


def both(oracle, data, file_size=None):
    c, o = c_parse(data, file_size), o_parse(oracle, data, file_size)
    assert c == o, (c, o)
    return c


# ---- the reference's cases (root.zig:320-439)

def test_accepts_two_contiguous_tensors(ncm, oracle):
    r = both(oracle, make_file('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},\n'
                               ' "b":{"dtype":"BF16","shape":[2,2],"data_offsets":[8,16]}}', 16))
    assert r[0] == "ok" and len(r[3]) == 2 and r[2] == 16 and r[3][1][1] == "BF16"


def test_sorts_tensors_by_offset(ncm, oracle):
    r = both(oracle, make_file('{"b":{"dtype":"F32","shape":[1],"data_offsets":[4,8]},\n'
                               ' "a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', 8))
    assert r[3][0][0] == "a"


@pytest.mark.parametrize("js,data_len,err", [
    ('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},\n'
     ' "b":{"dtype":"F32","shape":[1],"data_offsets":[8,12]}}', 12, "InvalidOffsets"),
    ('{"a":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}', 8, "SizeMismatch"),
    ('{"a":{"dtype":"F7","shape":[1],"data_offsets":[0,1]}}', 1, "UnknownDtype"),
    ('{"a":{"dtype":"F4","shape":[3],"data_offsets":[0,2]}}', 2, "MisalignedBits"),
    ('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', 8, "FileSizeMismatch"),
    ('{"__metadata__":{"count":1},"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}', 1,
     "InvalidHeader"),
])
def test_reference_rejections(ncm, oracle, js, data_len, err):
    assert both(oracle, make_file(js, data_len)) == ("err", err)


def test_string_metadata_accepted(ncm, oracle):
    r = both(oracle, make_file('{"__metadata__":{"format":"pt"},'
                               '"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}', 1))
    assert r[0] == "ok"


def test_header_longer_than_maximum(ncm, oracle):
    prefix = (100_000_000 + 1).to_bytes(8, "little")
    assert both(oracle, prefix) == ("err", "HeaderTooLarge")
    assert both(oracle, b"\x01\x02") == ("err", "HeaderTooSmall")
    assert both(oracle, (20).to_bytes(8, "little") + b"{}") == ("err", "InvalidHeaderLength")


def test_dtype_names_round_trip(ncm, oracle):
    L = ncm.lib()
    names = [L.ncm_st_dtype_name(i).decode() for i in range(22)]
    assert names == [n for n, _ in oracle.ST_DTYPES]
    assert names[18] == "BF16" and names[10] == "F6_E2M3"
    assert [L.ncm_st_dtype_bits(i) for i in range(22)] == [b for _, b in oracle.ST_DTYPES]
    # Names are case sensitive.
    assert both(oracle, make_file('{"a":{"dtype":"bf16","shape":[1],"data_offsets":[0,2]}}', 2)) \
        == ("err", "UnknownDtype")


def test_sharded_index(ncm, oracle):
    good = ('{"metadata":{"total_size":16},"weight_map":{"a":"model-00001-of-00002.safetensors",'
            '"b":"model-00002-of-00002.safetensors"}}')
    entries, total = st.parse_index(good)
    assert len(entries) == 2 and total == 16
    assert (entries, total) == oracle.st_parse_index(good)
    for bad, err in (('{"weight_map":{"a":"../escape.safetensors"}}', "UnsafeShardName"),
                     ('{"weight_map":{"a":"x\\\\y"}}', "UnsafeShardName"),
                     ('{"weight_map":{"a":".."}}', "UnsafeShardName"),
                     ('{"weight_map":{"a":1}}', "InvalidIndex"),
                     ('{"weight_map":[]}', "InvalidIndex"),
                     ('{"metadata":[],"weight_map":{}}', "InvalidIndex"),
                     ('{"metadata":{"total_size":-1},"weight_map":{}}', "InvalidHeader"),
                     ('[1]', "InvalidIndex"), ('{"weight_map":{}', "SyntaxError")):
        with pytest.raises(NcmError) as ei:
            st.parse_index(bad)
        assert ei.value.detail == err, bad
        with pytest.raises(oracle.StError) as eo:
            oracle.st_parse_index(bad)
        assert str(eo.value) == err
    assert st.parse_index('{"weight_map":{}}') == ([], None)


def _cut_at_nul(r):
    """A C string ends at U+0000: the C ABI's names read as cut there."""
    if r[0] != "ok":
        return r
    return r[:3] + ([(t[0].split("\0")[0],) + tuple(t[1:]) for t in r[3]],)


def test_names_holding_nul(ncm, oracle):
    """A "\\u0000" escape in a tensor name or index key is a character of the
    key (the reference's JSON strings are byte slices). Repeated keys are
    matched whole, so "a\\u0000b" and "a" are two tensors, and a repeated
    "a\\u0000" keeps its last value (these inputs once made the reader
    dereference a failed lookup)."""
    js = ('{"a\\u0000b":{"dtype":"U8","shape":[1],"data_offsets":[0,1]},'
          '"a":{"dtype":"U8","shape":[2],"data_offsets":[1,3]}}')
    data = make_file(js, 3)
    c = c_parse(data)
    assert c == _cut_at_nul(o_parse(oracle, data))
    assert [t[2] for t in c[3]] == [[1], [2]]
    f = st.SafetensorsFile(data=data)
    assert f.find("a").shape == (2,)  # the whole-name match, not "a\0b"
    f.close()
    js2 = ('{"a\\u0000":{"dtype":"U8","shape":[9],"data_offsets":[0,9]},'
           '"a\\u0000":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}')
    data2 = make_file(js2, 1)
    c2 = c_parse(data2)
    assert c2 == _cut_at_nul(o_parse(oracle, data2)) and c2[3][0][2] == [1]

    ix = '{"weight_map":{"a\\u0000b":"s1.safetensors","a":"s2.safetensors"}}'
    entries, _ = st.parse_index(ix)
    want, _ = oracle.st_parse_index(ix)
    assert entries == [(k.split("\0")[0], v) for k, v in want] and len(entries) == 2
    ix2 = '{"weight_map":{"a\\u0000":"s1.safetensors","a\\u0000":"s2.safetensors"}}'
    assert st.parse_index(ix2)[0] == [("a", "s2.safetensors")]
    assert oracle.st_parse_index(ix2)[0] == [("a\0", "s2.safetensors")]


# ---- generated headers: the C parser and the oracle agree on every outcome

def _random_header(rng):
    dts = ["BOOL", "U8", "I16", "F4", "F6_E2M3", "F8_E4M3", "F16", "BF16", "F32", "F64", "C64"]
    bits = {"BOOL": 8, "U8": 8, "I16": 16, "F4": 4, "F6_E2M3": 6, "F8_E4M3": 8, "F16": 16,
            "BF16": 16, "F32": 32, "F64": 64, "C64": 64}
    n = rng.randint(0, 5)
    entries, off = [], 0
    for i in range(n):
        dt = rng.choice(dts)
        shape = [rng.randint(0, 5) for _ in range(rng.randint(0, 3))]
        cnt = 1
        for d in shape:
            cnt *= d
        size = (cnt * bits[dt] + 7) // 8
        entries.append([f"t{i}", {"dtype": dt, "shape": shape, "data_offsets": [off, off + size]}])
        off += size
    rng.shuffle(entries)
    if rng.random() < 0.3:
        entries.insert(rng.randint(0, len(entries)), ["__metadata__", {"format": "pt"}])
    return entries, off


def _mutate(rng, entries, data_len):
    kind = rng.randint(0, 14)
    tensors = [e for e in entries if e[0] != "__metadata__"]
    t = rng.choice(tensors)[1] if tensors else None
    if kind == 0 and t:
        t["data_offsets"][1] += rng.choice([-1, 1, 8])
    elif kind == 1 and t:
        t["data_offsets"] = [t["data_offsets"][0] + 1, t["data_offsets"][1] + 1]
    elif kind == 2 and t:
        t["dtype"] = rng.choice(["F7", "bf16", "", "FLOAT"])
    elif kind == 3 and t:
        t["shape"] = [rng.choice([1.0, -1, "2", True, None, 2**63, 2**64])]
    elif kind == 4 and t:
        del t[rng.choice(["dtype", "shape", "data_offsets"])]
    elif kind == 5 and t:
        t["data_offsets"] = t["data_offsets"][:1]
    elif kind == 6:
        entries.insert(0, ["__metadata__", rng.choice([{"n": 1}, [], "x", {"a": None}])])
    elif kind == 7 and t:
        t["shape"] = [2**40, 2**40]
    elif kind == 8:
        data_len += rng.choice([-1, 1])
    elif kind == 9 and t:
        t["extra"] = {"ignored": [1, 2, {"x": 1.5}]}
    elif kind == 10 and entries:
        entries.append([entries[0][0], entries[0][1]])  # repeated key
    elif kind == 11 and t:
        t["data_offsets"] = [t["data_offsets"][1], t["data_offsets"][0]]
    elif kind == 12 and t:
        t["dtype"] = 18
    return entries, data_len, kind


def _encode(rng, entries, kind):
    body = ",".join(json.dumps(k) + ":" + json.dumps(v) for k, v in entries)
    text = "{" + body + "}"
    if kind == 13:
        text = rng.choice([text + " x", text[:-1], text.replace(":", " : ") + "\n", "[" + text + "]",
                           text.replace("{", "{ ", 1), "﻿" + text, text + ",", "nul" + text])
    raw = text.encode("utf-8")
    if kind == 14:
        raw = raw.replace(b"t", rng.choice([b"\xff", b"\xc0\xaf", b"\xed\xa0\x80", b"t"]), 1)
    return raw


def test_generated_headers_match_oracle(ncm, oracle):
    rng = random.Random(2026)
    outcomes = {}
    for _ in range(3000):
        entries, data_len = _random_header(rng)
        kind = -1
        if rng.random() < 0.7:
            entries, data_len, kind = _mutate(rng, entries, data_len)
        raw = _encode(rng, entries, kind)
        if data_len < 0:
            continue
        data = len(raw).to_bytes(8, "little") + raw + bytes(data_len)
        r = both(oracle, data)
        outcomes[r[1] if r[0] == "err" else "ok"] = outcomes.get(r[1] if r[0] == "err" else "ok", 0) + 1
    # The generator reaches every outcome that it targets.
    for name in ("ok", "InvalidOffsets", "SizeMismatch", "UnknownDtype", "InvalidHeader",
                 "ShapeOverflow", "FileSizeMismatch", "SyntaxError", "InvalidUtf8",
                 "MisalignedBits"):
        assert outcomes.get(name, 0) > 0, (name, outcomes)
