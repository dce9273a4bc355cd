"""The desc-v1 reader and its JSON layer against the reference's own (ss_desc_from_json / ss_desc_to_json of
oracle/_ref, compiled from its sources), on the CPU: for each document both accept it and write the same canonical
bytes, or both refuse it with the same status.

Documents: valid random descriptors with one mutation each (a key removed, an unknown or "x-" key added, a value of
the wrong type, out of range, inconsistent with another - the rules of reference src/desc.cpp:128-413), and JSON text
edge cases (escapes, surrogates, raw control and non-ASCII bytes, number forms, whitespace, nesting depth, truncation,
duplicates, trailing text; reference src/json.cpp)."""
import ctypes as C
import json
import zlib

import numpy as np
import pytest

from oracle import ref
from tierstream_amd import ss

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (needs the reference sources)")
vp = C.c_void_p


def _canon(L, text: bytes):
    d = vp()
    st = L.ss_desc_from_json(text, len(text), C.byref(d))
    if st != 0:
        return st, None
    try:
        s, n = C.c_char_p(), C.c_size_t()
        assert L.ss_desc_to_json(d, C.byref(s), C.byref(n)) == 0
        out = C.string_at(s, n.value)
        L.ss_free(s)
        return 0, out
    finally:
        L.ss_desc_free(d)


def _both(text: bytes):
    return _canon(ss._declare(), text), _canon(ref.lib(), text)


def _base(rng):
    layers, off = [], 0
    kinds = ["dense"] + list(rng.choice(["moe", "moe", "blob"], size=int(rng.integers(2, 5))))
    for i, kind in enumerate(kinds):
        if kind == "dense":
            layers.append({"index": i, "kind": "dense", "fixed_bytes": int(rng.integers(0, 1 << 20))})
            continue
        n = 1 if kind == "blob" else int(rng.choice([2, 4, 8]))
        parts, po = [], 0
        n_parts = int(rng.integers(1, 4))
        pb = [int(rng.choice([1, 3, 64])) * 4096 for _ in range(n_parts)]
        stride = (sum(pb) + 4095) // 4096 * 4096
        for p, b in enumerate(pb):
            parts.append({"name": f"w{p}", "format": str(rng.choice(["BF16", "Q4_K", "U8", "x-mine"])), "source": 0,
                          "offset": off + po, "stride": stride, "bytes": b})
            po += b
        lay = {"index": i, "kind": kind, "n_units": n, "parts": parts,
               "hash": [f"{int(h):016x}" for h in rng.integers(0, 2**63, size=n)]}
        if kind == "moe":
            lay["top_k"] = int(rng.integers(1, n + 1))
            if rng.random() < 0.5:
                lay["router"] = {"tensor": f"blk.{i}.gate", "rows": n, "cols": 64}
        if rng.random() < 0.3:
            lay["benefit"] = [float(v) for v in rng.random(n)]
        layers.append(lay)
        off += n * stride
    return {"schema": "strix-stream/desc-v1", "model": "m", "engine": "e", "unit_align": 256,
            "sources": [{"name": "w", "path": "/nonexistent/w.bin", "align": 4096}], "layers": layers}


def _pick(rng, d, kind=None):
    c = [l for l in d["layers"] if kind is None or l["kind"] == kind]
    return c[int(rng.integers(len(c)))] if c else None


def _units(d):
    return [l for l in d["layers"] if l.get("n_units", 0)]


# one mutation each: (name, fn(d, rng))
def _set(path_fn, value):
    def f(d, rng):
        obj, key = path_fn(d, rng)
        if obj is not None:
            obj[key] = value
    return f


def _del(path_fn):
    def f(d, rng):
        obj, key = path_fn(d, rng)
        if obj is not None:
            obj.pop(key, None)
    return f


def top(k):
    return lambda d, rng: (d, k)


def lay(k, kind=None):
    return lambda d, rng: ((_pick(rng, d, kind)), k)


def part(k):
    def f(d, rng):
        l = _pick(rng, {"layers": _units(d)})
        return (l["parts"][int(rng.integers(len(l["parts"])))], k) if l else (None, k)
    return f


def src(k):
    return lambda d, rng: (d["sources"][0], k)


def _router(k):
    def f(d, rng):
        l = _pick(rng, d, "moe")
        if l is None:
            return None, k
        l.setdefault("router", {"tensor": "g", "rows": l["n_units"], "cols": 8})
        return l["router"], k
    return f


def _swap_layers(d, rng):
    d["layers"][0], d["layers"][1] = d["layers"][1], d["layers"][0]


def _dense_with_parts(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["kind"] = "dense"


def _dense_clean(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    for k in ["n_units", "parts", "top_k", "hash", "benefit", "router"]:
        l.pop(k, None)
    l["kind"] = "dense"


def _top_k_over(d, rng):
    l = _pick(rng, d, "moe")
    if l:
        l["top_k"] = l["n_units"] + 1


def _unit_bytes_wrong(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["unit_bytes"] = sum(p["bytes"] for p in l["parts"]) + 1


def _unit_bytes_right(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["unit_bytes"] = sum(p["bytes"] for p in l["parts"])


def _hash_short(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["hash"] = l["hash"][:-1]


def _hash_upper(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["hash"][0] = l["hash"][0].upper() if any(c in "abcdef" for c in l["hash"][0]) else "ABCDEF0123456789"


def _hash_15(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["hash"][0] = l["hash"][0][:15]


def _benefit_len(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["benefit"] = [0.5] * (l["n_units"] + 1)


def _benefit_str(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["benefit"] = ["x"] * l["n_units"]


def _router_rows(d, rng):
    l = _pick(rng, d, "moe")
    if l:
        l["router"] = {"tensor": "g", "rows": l["n_units"] + 1}


def _stride_short(d, rng):
    l = _pick(rng, d, "moe")
    if l:
        l["parts"][0]["stride"] = l["parts"][0]["bytes"] - 1


def _stride_absent(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["parts"][0].pop("stride", None)


def _offset_overflow(d, rng):
    l = _pick(rng, d, "moe")
    if l:
        l["parts"][0]["offset"] = 2**64 - 4096


def _huge_total(d, rng):
    l = _pick(rng, d, "moe")
    if l:
        l["n_units"], l["top_k"] = 64, 1
        l.pop("hash", None), l.pop("benefit", None), l.pop("router", None)
        l["parts"] = [{"format": "U8", "offset": 0, "stride": 2**50, "bytes": 2**50}]


def _fixed_overflow(d, rng):
    d["fixed_device"] = [{"name": "a", "bytes": 2**63}, {"name": "b", "bytes": 2**63}]


def _host_fixed_ok(d, rng):
    d["host_fixed"] = [{"name": "emb", "bytes": 12345}]


def _lookup(placement):
    def f(d, rng):
        d["lookup_tables"] = [{"name": "tok", "source": 0, "offset": 4096, "rows": 10, "row_bytes": 64,
                               "placement": placement}]
    return f


def _lookup_src(d, rng):
    d["lookup_tables"] = [{"name": "tok", "source": 3, "rows": 10, "row_bytes": 64}]


def _lookup_missing(d, rng):
    d["lookup_tables"] = [{"name": "tok", "rows": 10}]


def _no_sources(d, rng):
    d["sources"] = []


def _two_sources(d, rng):
    d["sources"].append({"path": "/nonexistent/b.bin"})
    l = _pick(rng, {"layers": _units(d)})
    l["parts"][0]["source"] = 1


def _parts_empty(d, rng):
    l = _pick(rng, {"layers": _units(d)})
    l["parts"] = []


def _fixed_bytes_layer(d, rng):
    l = _pick(rng, d)
    l["fixed_bytes"] = 2**64 - 1


MUTATIONS = [
    ("none", lambda d, rng: None),
    ("schema-missing", _del(top("schema"))), ("schema-renamed", _set(top("schema"), "tierstream/desc-v1")),
    ("schema-v2", _set(top("schema"), "strix-stream/desc-v2")), ("schema-num", _set(top("schema"), 1)),
    ("model-num", _set(top("model"), 5)), ("model-unicode", _set(top("model"), "modéle ☃ \U0001F600")),
    ("model-escapes", _set(top("model"), "a\"b\\c\n\t\x01\x1f/")), ("engine-empty", _set(top("engine"), "")),
    ("routes", _set(top("routes"), "routes.bin")), ("routes-num", _set(top("routes"), 3)),
    ("align-0", _set(top("unit_align"), 0)), ("align-3", _set(top("unit_align"), 3)),
    ("align-4096", _set(top("unit_align"), 4096)), ("align-str", _set(top("unit_align"), "256")),
    ("align-float", _set(top("unit_align"), 256.0)), ("align-neg", _set(top("unit_align"), -256)),
    ("ring-max", _set(top("ring_slots"), 1 << 20)), ("ring-over", _set(top("ring_slots"), (1 << 20) + 1)),
    ("order-prefix", _set(top("order"), "prefix")), ("order-bad", _set(top("order"), "random")),
    ("tiers-disk", _set(top("tiers"), "disk")), ("tiers-pair", _set(top("tiers"), "pair")),
    ("tiers-pinned", _set(top("tiers"), "pinned")), ("tiers-bad", _set(top("tiers"), "hbm")),
    ("state-neg", _set(top("state_bytes_per_position"), -1)), ("state-frac", _set(top("state_bytes_per_position"), 1.5)),
    ("ws-max", _set(top("workspace_bytes_per_row"), 2**64 - 1)), ("ws-over", _set(top("workspace_bytes_per_row"), 2**64)),
    ("fixed-device", _set(top("fixed_device"), [{"name": "a", "bytes": 5}])),
    ("fixed-device-nobytes", _set(top("fixed_device"), [{"name": "a"}])),
    ("fixed-device-obj", _set(top("fixed_device"), {})),
    ("host-fixed-extra", _set(top("host_fixed"), [{"name": "a", "bytes": 5, "extra": 1}])),
    ("host-fixed-ok", _host_fixed_ok), ("fixed-overflow", _fixed_overflow),
    ("lookup-file", _lookup("file")), ("lookup-device", _lookup("device")), ("lookup-gpu", _lookup("gpu")),
    ("lookup-src", _lookup_src), ("lookup-missing", _lookup_missing),
    ("no-sources", _no_sources), ("two-sources", _two_sources), ("src-align-3", _set(src("align"), 3)),
    ("src-align-2M", _set(src("align"), 2 << 20)), ("src-align-1M", _set(src("align"), 1 << 20)),
    ("src-no-path", _del(src("path"))), ("src-extra", _set(src("mode"), "r")), ("src-x", _set(src("x-mode"), "r")),
    ("x-note", _set(top("x-note"), {"a": [1, 2, {"b": None}]})), ("unknown-top", _set(top("bogus"), 1)),
    ("layers-empty", _set(top("layers"), [])), ("layers-obj", _set(top("layers"), {})), ("layers-missing", _del(top("layers"))),
    ("swap-layers", _swap_layers), ("index-neg", _set(lay("index"), -1)), ("index-4096", _set(lay("index"), 4096)),
    ("index-str", _set(lay("index"), "0")), ("kind-bad", _set(lay("kind"), "conv")), ("kind-missing", _del(lay("kind"))),
    ("dense-with-parts", _dense_with_parts), ("dense-clean", _dense_clean),
    ("blob-2", _set(lay("n_units", "blob"), 2)), ("units-over", _set(lay("n_units", "moe"), 65537)),
    ("units-0-moe", _set(lay("n_units", "moe"), 0)), ("topk-0", _set(lay("top_k", "moe"), 0)), ("topk-over", _top_k_over),
    ("shared", _set(lay("n_shared", "moe"), 2)), ("shared-over", _set(lay("n_shared", "moe"), 65537)),
    ("unit-bytes-wrong", _unit_bytes_wrong), ("unit-bytes-right", _unit_bytes_right),
    ("hash-short", _hash_short), ("hash-upper", _hash_upper), ("hash-15", _hash_15),
    ("hash-num", _set(lay("hash", "moe"), [1, 2])), ("hash-obj", _set(lay("hash", "moe"), {})),
    ("benefit-len", _benefit_len), ("benefit-str", _benefit_str),
    ("streamable-false", _set(lay("streamable", "moe"), False)), ("streamable-str", _set(lay("streamable", "moe"), "no")),
    ("router-rows", _router_rows), ("router-no-tensor", _del(_router("tensor"))), ("router-extra", _set(_router("gain"), 1)),
    ("router-cols-over", _set(_router("cols"), (1 << 24) + 1)), ("router-bias", _set(_router("bias"), "b")),
    ("router-score", _set(_router("score"), "sigmoid")), ("router-format", _set(_router("format"), "BF16")),
    ("layer-extra", _set(lay("weights"), 1)), ("layer-x", _set(lay("x-src"), "gguf")),
    ("fixed-bytes-layer-max", _fixed_bytes_layer),
    ("part-bytes-0", _set(part("bytes"), 0)), ("part-format-bad", _set(part("format"), "FP7")),
    ("part-format-x", _set(part("format"), "x-packed")), ("part-format-mixed", _set(part("format"), "mixed")),
    ("part-format-missing", _del(part("format"))), ("part-offset-missing", _del(part("offset"))),
    ("part-bytes-missing", _del(part("bytes"))), ("part-source-1", _set(part("source"), 1)),
    ("part-source-over", _set(part("source"), 1025)), ("part-extra", _set(part("dtype"), "f")),
    ("part-name-missing", _del(part("name"))), ("stride-short", _stride_short), ("stride-absent", _stride_absent),
    ("offset-overflow", _offset_overflow), ("huge-total", _huge_total), ("parts-empty", _parts_empty),
    ("parts-obj", _set(lay("parts", "moe"), {})),
]


@pytest.mark.parametrize("name,fn", MUTATIONS, ids=[m[0] for m in MUTATIONS])
@pytest.mark.parametrize("seed", range(3))
def test_mutated_descriptor_matches_reference(name, fn, seed):
    rng = np.random.default_rng(seed * 1000 + zlib.crc32(name.encode()) % 1000)
    d = _base(rng)
    fn(d, rng)
    text = json.dumps(d, ensure_ascii=bool(seed % 2)).encode()
    (st_o, out_o), (st_t, out_t) = _both(text)
    assert st_o == st_t, (name, st_o, st_t, ref.lib().ss_last_error())
    assert out_o == out_t, name


def _doc(model_text: str = '"m"', extra: str = "", align: str = "256", ws: str = "") -> bytes:
    layer = ('{"index":0,"kind":"moe","n_units":2,"top_k":1,"parts":[{"format":"U8","offset":0,"bytes":4096}],'
             '"benefit":[0.25,1e-3]}')
    return (f'{ws}{{{ws}"schema"{ws}:{ws}"strix-stream/desc-v1",{ws}"model":{model_text},"unit_align":{align},'
            f'"sources":[{{"path":"/x"}}],"layers":[{layer}]{extra}{ws}}}{ws}').encode("utf-8", "surrogatepass")


SYNTAX = [
    ("plain", _doc()),
    ("esc-basic", _doc(r'"a\"b\\c\/d\b\f\n\r\t"')), ("esc-u", _doc(r'"\u00e9\u2603\u0041"')),
    ("esc-nul", _doc(r'"a\u0000b"')), ("esc-1f", _doc(r'"\u001f\u007f"')), ("esc-upper-hex", _doc(r'"\u00E9\uABCD"')),
    ("pair", _doc(r'"\ud83d\ude00"')), ("lone-low", _doc(r'"\udc00"')), ("lone-high", _doc(r'"\ud800"')),
    ("high-then-char", _doc(r'"\ud800x"')), ("high-then-bmp", _doc(r'"\ud800A"')),
    ("high-high", _doc(r'"\ud800\ud800"')), ("short-u", _doc(r'"\u00"')), ("bad-u", _doc(r'"\u00g0"')),
    ("bad-escape", _doc(r'"\x41"')), ("raw-ctrl", _doc('"a\x01b"')), ("raw-tab", _doc('"a\tb"')),
    ("raw-del", _doc('"a\x7fb"')), ("raw-utf8", _doc('"café ☃"')), ("unterminated", _doc('"abc')),
    ("num-plain", _doc(align="512")), ("num-exp", _doc(align="2.56e2")), ("num-frac", _doc(align="256.0")),
    ("num-lead0", _doc(align="0256")), ("num-neg", _doc(align="-256")), ("num-neg0", _doc(align="-0")),
    ("num-zero", _doc(align="0")), ("num-plus", _doc(align="+256")), ("num-dot", _doc(align="256.")),
    ("num-exp-sign", _doc(align="1E+2")), ("num-exp-empty", _doc(align="1e")),
    ("ws-mixed", _doc(ws=" \t\n\r ")), ("ws-formfeed", _doc(ws="\f")),
    ("trailing-x", _doc() + b"x"), ("trailing-ws", _doc() + b" \n"), ("trailing-comma", _doc(extra=",")),
    ("dup-key", _doc(extra=',"model":"n"')), ("x-null", _doc(extra=',"x-a":null')),
    ("x-bools", _doc(extra=',"x-a":[true,false,null]')), ("x-bad-literal", _doc(extra=',"x-a":nul')),
    ("x-True", _doc(extra=',"x-a":True')), ("x-missing-colon", _doc(extra=',"x-a" 1')),
    ("x-arr-trailing-comma", _doc(extra=',"x-a":[1,]')), ("x-empty-obj", _doc(extra=',"x-a":{}')),
    ("x-obj-num-key", _doc(extra=',"x-a":{1:2}')), ("x-big-num", _doc(extra=',"x-a":1e999999')),
    ("benefit-inf", _doc().replace(b"1e-3", b"1e400")), ("benefit-tiny", _doc().replace(b"1e-3", b"1e-400")),
    ("benefit-int", _doc().replace(b"1e-3", b"7")), ("benefit-neg", _doc().replace(b"1e-3", b"-0.5")),
    ("empty", b""), ("only-ws", b"  \n"), ("top-array", b"[]"), ("top-string", b'"x"'), ("truncated", _doc()[:-7]),
]
for n in range(61, 66):
    SYNTAX.append((f"depth-{n}", _doc(extra=',"x-d":' + "[" * n + "]" * n)))
    SYNTAX.append((f"depth-{n}-leaf", _doc(extra=',"x-d":' + "[" * n + "1" + "]" * n)))
    SYNTAX.append((f"depth-{n}-obj", _doc(extra=',"x-d":' + '{"a":' * n + "0" + "}" * n)))


@pytest.mark.parametrize("name,text", SYNTAX, ids=[s[0] for s in SYNTAX])
def test_json_text_matches_reference(name, text):
    (st_o, out_o), (st_t, out_t) = _both(text)
    assert st_o == st_t, (name, st_o, st_t, ref.lib().ss_last_error())
    assert out_o == out_t, name


def test_cases_cover_both_outcomes():
    """The grid is not vacuous: many mutated documents are accepted (canonical bytes compared) and many refused."""
    acc = ref_acc = 0
    for i, (name, fn) in enumerate(MUTATIONS):
        rng = np.random.default_rng(i)
        d = _base(rng)
        fn(d, rng)
        st, _ = _canon(ref.lib(), json.dumps(d).encode())
        acc += st == 0
    for name, text in SYNTAX:
        st, _ = _canon(ref.lib(), text)
        ref_acc += st == 0
    assert 25 < acc < len(MUTATIONS) - 30, acc
    assert 15 < ref_acc < len(SYNTAX) - 20, ref_acc
