"""The MLIR bytecode container reader behind PJRT_Client_Compile (a StableHLO
portable artifact is what jaxlib sends; the reference deserializes it with
the MLIR libraries, src/jam/parse.cc:53-63).

No MLIR writer and no artifact exist in this environment, so the streams are
assembled here, byte for byte, by the writer algorithm of MLIR's bytecode
format (magic, version, producer, sections with optional 0xCB alignment
padding, prefix varints with flags in the low bit, the string / dialect /
attribute-type-offset / IR / properties sections, isolated regions in nested
IR sections from version 2, use-list orders from version 3, elided unknown
block-argument locations and an op-name count from version 4, registered
flags on op names and op properties from version 5).  The reader's output
reaches the test through the compiled plan (a hand-assembled VHLO artifact
compiles to the plan of the same module as text) or through the named
compile error, which lists the dialects (with versions), the producer and
every operation of the tree.  CPU only."""

import struct

import pytest

from mi355x_pjrt import pjrt

# ------------------------------------------------------------------ writer


def varint(v, wide=False):
    """Prefix varint: n bytes hold ((v << 1) | 1) << (n - 1), little-endian;
    values needing more than 56 bits (or wide=True) are a 0 byte + 8 raw bytes."""
    if not wide:
        for n in range(1, 9):
            if v < (1 << (7 * n)):
                return (((v << 1) | 1) << (n - 1)).to_bytes(n, "little")
    return b"\x00" + struct.pack("<Q", v)


def vflag(v, f):
    return varint((v << 1) | int(bool(f)))


def section(sid, data, pos, align=1):
    """Section at stream offset `pos` (the alignment is of the data's offset)."""
    head = bytes([sid | (0x80 if align > 1 else 0)]) + varint(len(data))
    if align > 1:
        head += varint(align)
        while (pos + len(head)) % align:
            head += b"\xcb"
    return head + data


class Stream:
    def __init__(self, version, producer):
        self.version, self.producer = version, producer
        self.strings, self.dialects, self.op_names, self.attrs, self.types = [], [], [], [], []
        self.props = []

    def s(self, text):
        if text not in self.strings:
            self.strings.append(text)
        return self.strings.index(text)

    def dialect(self, name, version_varints=None):
        self.dialects.append((self.s(name), version_varints))
        return len(self.dialects) - 1

    def op_name(self, dialect, name, registered=True):
        self.op_names.append((dialect, self.s(name), registered))
        return len(self.op_names) - 1

    def attr(self, dialect, payload, custom):
        self.attrs.append((dialect, payload, custom))
        return len(self.attrs) - 1

    def type(self, dialect, payload, custom):
        self.types.append((dialect, payload, custom))
        return len(self.types) - 1

    def prop(self, payload):
        self.props.append(payload)
        return len(self.props) - 1

    # ---- IR
    def op(self, o):
        v = self.version
        out = varint(o["name"])
        mask = 0
        body = varint(o.get("loc", 0), wide=o.get("wide_loc", False))
        if o.get("attrs") is not None:
            mask |= 0x01
            body += varint(o["attrs"])
        if o.get("props") is not None:
            mask |= 0x40
            body += varint(o["props"])
        if o.get("results"):
            mask |= 0x02
            body += varint(len(o["results"])) + b"".join(varint(t) for t in o["results"])
        if o.get("operands"):
            mask |= 0x04
            body += varint(len(o["operands"])) + b"".join(varint(x) for x in o["operands"])
        if o.get("uselists"):
            mask |= 0x20
            body += self.uselists(o["uselists"], len(o.get("results", [])))
        regions = o.get("regions", [])
        tail = b""
        if regions:
            mask |= 0x10
            iso = o.get("isolated", False)
            tail += vflag(len(regions), iso)
            rbytes = b"".join(self.region(r) for r in regions)
            tail += section(4, rbytes, 0) if (iso and v >= 2) else rbytes
        return out + bytes([mask]) + body + tail

    def uselists(self, orders, nres):
        out = b"" if nres == 1 else varint(len(orders))
        for idx, perm in orders:
            if nres != 1:
                out += varint(idx)
            out += vflag(len(perm), False) + b"".join(varint(p) for p in perm)
        return out

    def region(self, r):
        if not r["blocks"]:
            return varint(0)
        return varint(len(r["blocks"])) + varint(r["num_values"]) + b"".join(self.block(b) for b in r["blocks"])

    def block(self, b):
        args = b.get("args", [])
        out = vflag(len(b["ops"]), bool(args))
        if args:
            out += varint(len(args))
            for ty, loc in args:
                if self.version >= 4:
                    out += vflag(ty, loc is not None) + (varint(loc) if loc is not None else b"")
                else:
                    out += varint(ty) + varint(loc or 0)
            if self.version >= 3:
                out += b"\x00"
        return out + b"".join(self.op(o) for o in b["ops"])

    # ---- whole stream
    def build(self, top_ops, align_ir=1):
        v = self.version
        out = b"ML\xefR" + varint(v) + self.producer.encode() + b"\x00"
        # dialects
        d = varint(len(self.dialects))
        for name, ver in self.dialects:
            if v < 1:
                d += varint(name)
            else:
                d += vflag(name, ver is not None)
                if ver is not None:
                    d += section(7, b"".join(varint(x) for x in ver), 0)
        if v >= 4:
            d += varint(len(self.op_names))
        groups = []
        for dl, sid, reg in self.op_names:
            if groups and groups[-1][0] == dl:
                groups[-1][1].append((sid, reg))
            else:
                groups.append((dl, [(sid, reg)]))
        for dl, items in groups:
            d += varint(dl) + varint(len(items))
            for sid, reg in items:
                d += vflag(sid, reg) if v >= 5 else varint(sid)
        # attributes and types
        data, offs = b"", varint(len(self.attrs)) + varint(len(self.types))
        for table in (self.attrs, self.types):
            gr = []
            for dl, payload, custom in table:
                if gr and gr[-1][0] == dl:
                    gr[-1][1].append((payload, custom))
                else:
                    gr.append((dl, [(payload, custom)]))
            for dl, items in gr:
                offs += varint(dl) + varint(len(items))
                for payload, custom in items:
                    payload = payload if custom else payload.encode() + b"\x00"
                    data += payload
                    offs += vflag(len(payload), custom)
        ir = vflag(len(top_ops), False) + b"".join(self.op(o) for o in top_ops)
        strs = varint(len(self.strings)) + b"".join(varint(len(x) + 1) for x in reversed(self.strings))
        strs += b"".join(x.encode() + b"\x00" for x in self.strings)
        for sid, payload, al in ((1, d, 1), (3, offs, 1), (2, data, 1), (4, ir, align_ir), (0, strs, 1)):
            out += section(sid, payload, len(out), al)
        if v >= 5:
            p = varint(len(self.props)) + b"".join(varint(len(x)) + x for x in self.props)
            out += section(8, p, len(out))
        return out


def svarint(v):
    """Signed varint: zigzag ((v << 1) ^ (v >> 63)), then a prefix varint."""
    z = ((v << 1) ^ (v >> 63)) & ((1 << 64) - 1)
    return varint(z, wide=z >= (1 << 56))


# VHLO type codes (f32, tensor, function) and the builtin attribute codes the
# artifacts below use (DictionaryAttr, StringAttr, UnknownLoc)
TY_F32, TY_TENSOR, TY_FUNCTION = 4, 20, 8
BI_DICT, BI_STRING, BI_UNKNOWN_LOC = 1, 2, 15
AT_STRING, AT_TYPE, AT_CMP_DIR, AT_CMP_TYPE = 13, 17, 2, 3   # decoded by name, not by code


def artifact_v1(f32_code=TY_F32, dim=4, module_level_extra=False):
    """A StableHLO portable artifact of `lambda a, b: a + b` over f32[4],
    assembled byte for byte: builtin.module { vhlo.func_v1 @main (isolated)
    { ^bb(%a, %b): vhlo.add_v1; vhlo.return_v1 } }, with VHLO's binary types
    (f32; tensor = {rank, zigzag dims, element}; function = {inputs,
    results}) and attributes (a builtin DictionaryAttr of builtin StringAttr
    names holding a string and a type attribute)."""
    st = Stream(1, "StableHLO_v1.0.0")
    builtin = st.dialect("builtin")
    vhlo = st.dialect("vhlo", [1, 0, 0])
    module = st.op_name(builtin, "module")
    func, add, ret = (st.op_name(vhlo, n) for n in ("func_v1", "add_v1", "return_v1"))
    loc = st.attr(builtin, varint(BI_UNKNOWN_LOC), True)
    k_ft = st.attr(builtin, varint(BI_STRING) + varint(st.s("function_type")), True)
    k_name = st.attr(builtin, varint(BI_STRING) + varint(st.s("sym_name")), True)
    f32 = st.type(vhlo, varint(f32_code), True)
    tensor = st.type(vhlo, varint(TY_TENSOR) + varint(1) + svarint(dim) + varint(f32), True)
    fty = st.type(vhlo, varint(TY_FUNCTION) + varint(2) + varint(tensor) * 2 + varint(1) + varint(tensor), True)
    v_name = st.attr(vhlo, varint(AT_STRING) + varint(st.s("main")), True)
    v_ft = st.attr(vhlo, varint(AT_TYPE) + varint(fty), True)
    fattrs = st.attr(builtin, varint(BI_DICT) + varint(2) + varint(k_ft) + varint(v_ft) + varint(k_name) +
                     varint(v_name), True)
    body = {"blocks": [{"args": [(tensor, loc), (tensor, loc)],
                        "ops": [{"name": add, "loc": loc, "results": [tensor], "operands": [0, 1]},
                                {"name": ret, "loc": loc, "operands": [2]}]}], "num_values": 3}
    fn = {"name": func, "loc": loc, "attrs": fattrs, "regions": [body], "isolated": True}
    ops = [fn]
    if module_level_extra:
        ops.append({"name": ret, "loc": loc})
    top = {"name": module, "loc": loc, "regions": [{"blocks": [{"ops": ops}], "num_values": 0}], "isolated": True}
    return st, top


ADD_TEXT = """func.func public @main(%a: tensor<4xf32>, %b: tensor<4xf32>) -> tensor<4xf32> {
  %0 = stablehlo.add %a, %b : tensor<4xf32>
  return %0 : tensor<4xf32>
}"""


@pytest.fixture(scope="module")
def client():
    p = pjrt.Plugin()
    c = p.client()
    yield c
    c.close()


def compile_error(client, blob):
    with pytest.raises(pjrt.PjrtError) as ei:
        client.compile(blob)
    assert ei.value.code == "INVALID_ARGUMENT"
    assert ei.value.message.startswith(("jam compile: jam: MLIR bytecode", "jam compile: jam: VHLO"))
    return ei.value.message


def plan_of(client, program):
    e = client.compile(program)
    try:
        return e.plan(), e.output_types(), e.output_shapes()
    finally:
        e.destroy()


def test_varint_encodings_fixed_by_the_format():
    # one byte: (v << 1) | 1; two bytes: ((v << 1) | 1) << 1, little-endian
    assert varint(0) == b"\x01" and varint(1) == b"\x03" and varint(127) == b"\xff"
    assert varint(128) == b"\x02\x02" and varint((1 << 14) - 1) == b"\xfe\xff"
    assert varint(1 << 14) == b"\x04\x00\x02"
    assert varint(5, wide=True) == b"\x00\x05" + b"\x00" * 7


def test_portable_artifact_v1_compiles(client):
    """The hand-assembled artifact of a + b compiles to the plan of the same
    module as text: one elementwise launch, f32[4] out."""
    st, top = artifact_v1()
    assert plan_of(client, st.build([top])) == plan_of(client, ADD_TEXT)
    assert "] ew" in plan_of(client, ADD_TEXT)[0]


def test_vhlo_decoding_errors_are_named(client):
    """What the decoder refuses names itself, with the container summary
    (producer, dialect versions, op histogram) after it."""
    cases = {
        "dynamic dim": (artifact_v1(dim=-(1 << 63)), "has a dynamic dimension"),
        "unknown type code": (artifact_v1(f32_code=200), "type code 200, which is not decoded"),
        "complex element": (artifact_v1(f32_code=1), "element type complex is not supported"),
        "module-level op": (artifact_v1(module_level_extra=True), "module-level operation vhlo.return_v1"),
    }
    for name, ((st, top), needle) in cases.items():
        msg = compile_error(client, st.build([top]))
        assert needle in msg, (name, msg)
        assert "artifact: MLIR bytecode v1 from 'StableHLO_v1.0.0', dialects builtin, vhlo 1.0.0" in msg, msg
        assert "vhlo.func_v1 x1" in msg


def test_compare_type_checks_the_element_codes(client):
    """compare_type must fit the operands' element type: SIGNED on f32
    operands means the element type codes were not read as written."""
    def artifact(cmp_type):
        st = Stream(1, "StableHLO_v1.0.0")
        builtin = st.dialect("builtin")
        vhlo = st.dialect("vhlo", [1, 0, 0])
        module = st.op_name(builtin, "module")
        func, cmp, ret = (st.op_name(vhlo, n) for n in ("func_v1", "compare_v1", "return_v1"))
        loc = st.attr(builtin, varint(BI_UNKNOWN_LOC), True)
        keys = {k: st.attr(builtin, varint(BI_STRING) + varint(st.s(k)), True)
                for k in ("compare_type", "comparison_direction", "function_type", "sym_name")}
        f32 = st.type(vhlo, varint(TY_F32), True)
        i1 = st.type(vhlo, varint(0), True)
        t = st.type(vhlo, varint(TY_TENSOR) + varint(1) + svarint(4) + varint(f32), True)
        tb = st.type(vhlo, varint(TY_TENSOR) + varint(1) + svarint(4) + varint(i1), True)
        fty = st.type(vhlo, varint(TY_FUNCTION) + varint(2) + varint(t) * 2 + varint(1) + varint(tb), True)
        v_name = st.attr(vhlo, varint(AT_STRING) + varint(st.s("main")), True)
        v_ft = st.attr(vhlo, varint(AT_TYPE) + varint(fty), True)
        v_dir = st.attr(vhlo, varint(AT_CMP_DIR) + varint(3), True)        # GT
        v_ct = st.attr(vhlo, varint(AT_CMP_TYPE) + varint(cmp_type), True)
        fattrs = st.attr(builtin, varint(BI_DICT) + varint(2) + varint(keys["function_type"]) + varint(v_ft) +
                         varint(keys["sym_name"]) + varint(v_name), True)
        cattrs = st.attr(builtin, varint(BI_DICT) + varint(2) + varint(keys["compare_type"]) + varint(v_ct) +
                         varint(keys["comparison_direction"]) + varint(v_dir), True)
        body = {"blocks": [{"args": [(t, loc), (t, loc)],
                            "ops": [{"name": cmp, "loc": loc, "attrs": cattrs, "results": [tb], "operands": [0, 1]},
                                    {"name": ret, "loc": loc, "operands": [2]}]}], "num_values": 3}
        fn = {"name": func, "loc": loc, "attrs": fattrs, "regions": [body], "isolated": True}
        top = {"name": module, "loc": loc, "regions": [{"blocks": [{"ops": [fn]}], "num_values": 0}],
               "isolated": True}
        return st.build([top])

    text = """func.func public @main(%a: tensor<4xf32>, %b: tensor<4xf32>) -> tensor<4xi1> {
  %0 = stablehlo.compare GT, %a, %b, FLOAT : (tensor<4xf32>, tensor<4xf32>) -> tensor<4xi1>
  return %0 : tensor<4xi1>
}"""
    assert plan_of(client, artifact(1)) == plan_of(client, text)  # FLOAT
    assert "compare_type SIGNED on f32 operands" in compile_error(client, artifact(3))


def test_newest_layout_features(client):
    """Version 6: lazily loadable isolated regions (nested IR section), an
    aligned IR section with 0xCB padding, use-list orders on a two-result op
    and on block arguments, elided unknown block-argument locations, the
    op-name count, registered flags, properties, and a wide (9-byte) varint."""
    st = Stream(6, "MLIR21")
    builtin = st.dialect("builtin")
    t = st.dialect("test", [7])
    module = st.op_name(builtin, "module")
    two = st.op_name(t, "two_results")
    use = st.op_name(t, "use", registered=False)
    loc = st.attr(builtin, "loc(unknown)", False)
    i32 = st.type(builtin, "i32", False)
    pr = st.prop(b"\x01\x02\x03")
    blk = {"args": [(i32, None), (i32, 0)],
           "ops": [{"name": two, "loc": loc, "results": [i32, i32], "operands": [0, 1], "props": pr,
                    "uselists": [(0, [1, 0])]},
                   {"name": use, "loc": loc, "operands": [2, 2]},
                   {"name": use, "loc": loc, "operands": [3], "wide_loc": True}]}
    top = {"name": module, "loc": loc, "regions": [{"blocks": [blk], "num_values": 4}], "isolated": True}
    blob = st.build([top], align_ir=8)
    msg = compile_error(client, blob)
    assert "holds no vhlo dialect" in msg  # read in full, then refused: not an artifact
    assert "MLIR bytecode v6 from 'MLIR21'" in msg and "test 7" in msg
    assert "ops builtin.module x1, test.two_results x1, test.use x2" in msg


def test_malformed_streams_get_named_errors(client):
    st, top = artifact_v1()
    good = st.build([top])
    cases = {
        "truncated": (good[:-5], "unexpected end of data"),
        "newer": (good[:4] + varint(7) + good[5:], "newer than this reader"),
    }
    for name, (blob, needle) in cases.items():
        msg = compile_error(client, blob)
        assert needle in msg, (name, msg)
    # a section aligned with a padding byte other than 0xCB
    st2 = Stream(1, "p")
    b_ = st2.dialect("builtin")
    m_ = st2.op_name(b_, "module")
    l_ = st2.attr(b_, "loc(unknown)", False)
    blob = bytearray(st2.build([{"name": m_, "loc": l_}], align_ir=16))
    pad = blob.index(b"\xcb")
    blob[pad] = 0xCC
    assert "padding byte is not 0xCB" in compile_error(client, bytes(blob))
    # an operation naming an op-name index that does not exist
    st3 = Stream(1, "p")
    b3 = st3.dialect("builtin")
    st3.op_name(b3, "module")
    l3 = st3.attr(b3, "loc(unknown)", False)
    assert "operation name index out of range" in compile_error(client, st3.build([{"name": 5, "loc": l3}]))
    # the IR section missing altogether
    st4 = Stream(1, "p")
    b4 = st4.dialect("builtin")
    st4.op_name(b4, "module")
    st4.attr(b4, "loc(unknown)", False)
    full = st4.build([])
    ir_at = full.index(b"\x04" + varint(len(vflag(0, False))) + vflag(0, False))
    cut = full[:ir_at] + full[ir_at + 3:]
    assert "missing section id 4" in compile_error(client, cut)
