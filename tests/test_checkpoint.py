"""The .aic checkpoint format on the CPU (no GPU needed): the library's writer and reader
against an independent Python restatement of the reference's format
(src/train/checkpoint.cpp:30-186, docs/architecture.md:96-117) built on struct and
zlib.adler32, the corruption checks of tests/unit/test_train.cpp:92-122, and the
named_parameters() order of include/nn/module.hpp:63-76 as a tree walk."""
import ctypes as C
import os
import struct
import zlib

import numpy as np
import pytest

from autonomousaicore_amd import _lib

IO_ERROR, FORMAT_ERROR = 10, 11  # the reference's ErrorCode numbering (include/core/error.hpp:15-29)


def py_write(path, step, epoch, loss, desc, tensors):
    """tensors: (name, dims, dtype code, bytes)."""
    out = struct.pack("<IIqqfI", 0x41494330, 1, step, epoch, loss, len(desc)) + desc.encode()
    out += struct.pack("<Q", len(tensors))
    for name, dims, dt, data in tensors:
        out += struct.pack("<I", len(name)) + name.encode() + struct.pack("<i", len(dims))
        out += b"".join(struct.pack("<q", d) for d in dims)
        out += struct.pack("<iQ", dt, len(data)) + data + struct.pack("<I", zlib.adler32(data))
    with open(path, "wb") as f:
        f.write(out)


def py_read(path):
    b = open(path, "rb").read()
    magic, ver, step, epoch, loss, dl = struct.unpack_from("<IIqqfI", b, 0)
    o = 32
    desc = b[o:o + dl].decode()
    o += dl
    (n,) = struct.unpack_from("<Q", b, o)
    o += 8
    ts = []
    for _ in range(n):
        (nl,) = struct.unpack_from("<I", b, o)
        o += 4
        name = b[o:o + nl].decode()
        o += nl
        (rank,) = struct.unpack_from("<i", b, o)
        o += 4
        dims = list(struct.unpack_from(f"<{rank}q", b, o))
        o += 8 * rank
        dt, nb = struct.unpack_from("<iQ", b, o)
        o += 12
        data = b[o:o + nb]
        o += nb
        (ck,) = struct.unpack_from("<I", b, o)
        o += 4
        assert ck == zlib.adler32(data)
        ts.append((name, dims, dt, data))
    assert o == len(b)
    return (magic, ver, step, epoch, loss, desc), ts


def lib_write(path, step, epoch, loss, desc, tensors):
    n = len(tensors)
    names = (C.c_char_p * n)(*[t[0].encode() for t in tensors])
    ranks = (C.c_int32 * n)(*[len(t[1]) for t in tensors])
    flat = [d for t in tensors for d in t[1]]
    dims = (C.c_int64 * max(1, len(flat)))(*flat)
    dts = (C.c_int32 * n)(*[t[2] for t in tensors])
    bufs = [C.create_string_buffer(t[3], len(t[3])) for t in tensors]
    data = (C.c_void_p * n)(*[C.cast(bf, C.c_void_p) for bf in bufs])
    nb = (C.c_uint64 * n)(*[len(t[3]) for t in tensors])
    return _lib.load().aic_checkpoint_write(path.encode(), step, epoch, loss, desc.encode(), n, names, ranks, dims,
                                            dts, data, nb)


def lib_verify(path):
    n, step, epoch, loss = C.c_int64(), C.c_int64(), C.c_int64(), C.c_float()
    rc = _lib.load().aic_checkpoint_verify(path.encode(), C.byref(n), C.byref(step), C.byref(epoch), C.byref(loss))
    return rc, (n.value, step.value, epoch.value, loss.value)


def sample_tensors():
    rng = np.random.default_rng(5)
    return [("empty", [0, 3], 0, b""),
            ("optimizer.step", [1], 4, np.array([7], np.int64).tobytes()),
            ("norm.weight", [8], 0, np.ones(8, np.float32).tobytes()),
            ("layers.0.attn.q_proj.weight", [8, 8], 0, rng.standard_normal((8, 8)).astype(np.float32).tobytes())]


def test_writer_is_byte_identical_to_the_format(tmp_path):
    a, b = str(tmp_path / "lib.aic"), str(tmp_path / "py.aic")
    ts = sample_tensors()
    assert lib_write(a, 42, 2, 1.234, "unit_test_checkpoint", ts) == 0
    py_write(b, 42, 2, 1.234, "unit_test_checkpoint", ts)
    assert open(a, "rb").read() == open(b, "rb").read()
    head, back = py_read(a)
    assert head == (0x41494330, 1, 42, 2, pytest.approx(1.234), "unit_test_checkpoint")
    assert back == [(n, d, t, x) for n, d, t, x in ts]


def test_adler32_known_answer(tmp_path):
    # "Wikipedia" -> 0x11E60398 (the standard Adler-32 example); the file stores it after the data
    p = str(tmp_path / "w.aic")
    assert lib_write(p, 0, 0, 0.0, "", [("x", [9], 5, b"Wikipedia")]) == 0
    assert open(p, "rb").read()[-4:] == struct.pack("<I", 0x11E60398)
    assert zlib.adler32(b"Wikipedia") == 0x11E60398


def test_reader_accepts_the_format_and_checks_everything(tmp_path):
    p = str(tmp_path / "py.aic")
    ts = sample_tensors()
    py_write(p, 3, 1, 0.5, "d", ts)
    rc, (n, step, epoch, loss) = lib_verify(p)
    assert rc == 0 and (n, step, epoch, loss) == (4, 3, 1, 0.5)
    raw = bytearray(open(p, "rb").read())
    # a flipped payload byte near the end (tests/unit/test_train.cpp:104-116)
    bad = bytearray(raw)
    bad[-20] ^= 0xFF
    open(p, "wb").write(bytes(bad))
    assert lib_verify(p)[0] == FORMAT_ERROR
    assert "Adler-32" in _lib.load().aic_hip_last_error().decode()
    bad = bytearray(raw)
    bad[0] ^= 1                                   # magic
    open(p, "wb").write(bytes(bad))
    assert lib_verify(p)[0] == FORMAT_ERROR
    bad = bytearray(raw)
    bad[4] = 2                                    # version
    open(p, "wb").write(bytes(bad))
    assert lib_verify(p)[0] == FORMAT_ERROR
    open(p, "wb").write(bytes(raw[:-7]))          # truncated
    assert lib_verify(p)[0] == FORMAT_ERROR
    assert lib_verify(str(tmp_path / "missing.aic"))[0] == IO_ERROR


# --------------------------------------------------------------------- named_parameters order
def tree_order(names):
    """Module::named_parameters() as a walk over the module tree: at each module its own
    parameters (sorted), then its submodules (sorted by registered key, recursively)."""
    def keys(name):
        parts, out, i = name.split("."), [], 0
        while i < len(parts):
            if parts[i] in ("layers", "experts") and i + 1 < len(parts) and parts[i + 1].isdigit():
                out.append(parts[i] + "." + parts[i + 1])
                i += 2
            else:
                out.append(parts[i])
                i += 1
        return out

    root = {}
    for n in names:
        node = root
        ks = keys(n)
        for k in ks[:-1]:
            node = node.setdefault(("mod", k), {})
        node[("par", ks[-1])] = n

    def walk(node):
        out = [node[k] for k in sorted(k for k in node if k[0] == "par")]
        for k in sorted(k for k in node if k[0] == "mod"):
            out += walk(node[k])
        return out
    return walk(root)


def lm_names(L, experts=0, lora=False, tied=False):
    names = ["tok_embeddings.weight", "norm.weight"] + ([] if tied else ["lm_head.weight"])
    for l in range(L):
        p = f"layers.{l}."
        names += [p + "norm1.weight", p + "norm2.weight"]
        projs = ["attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.out_proj"]
        if experts:
            names.append(p + "moe.router.gate.weight")
            for e in range(experts):
                names += [p + f"moe.experts.{e}.{w}_proj.weight" for w in ("gate", "up", "down")]
        else:
            projs += ["ffn.gate_proj", "ffn.up_proj", "ffn.down_proj"]
        for q in projs:
            names.append(p + q + ".weight")
            if lora:
                names += [p + q + ".lora_A", p + q + ".lora_B"]
    return names


def lib_order(names):
    n = len(names)
    arr = (C.c_char_p * n)(*[x.encode() for x in names])
    out = (C.c_int64 * n)()
    assert _lib.load().aic_checkpoint_module_order(n, arr, out) == 0
    return [names[i] for i in out]


@pytest.mark.parametrize("kw", [dict(L=12), dict(L=2, tied=True), dict(L=3, experts=12), dict(L=2, lora=True)])
def test_module_order_matches_the_tree_walk(kw):
    names = lm_names(**kw)
    rng = np.random.default_rng(len(names))
    shuffled = [names[i] for i in rng.permutation(len(names))]
    want = tree_order(shuffled)
    assert lib_order(shuffled) == want
    # spot checks of the reference's order: layers.10 before layers.2, k_proj first in attn,
    # lora_A / lora_B before weight, experts.10 before experts.2
    if kw.get("L", 0) > 10:
        assert want.index("layers.10.attn.k_proj.weight") < want.index("layers.2.attn.k_proj.weight")
    assert want[0].startswith("layers.0.attn.k_proj")
    if kw.get("lora"):
        assert want[:3] == ["layers.0.attn.k_proj.lora_A", "layers.0.attn.k_proj.lora_B",
                            "layers.0.attn.k_proj.weight"]
    if kw.get("experts"):
        assert want.index("layers.0.moe.experts.10.down_proj.weight") < \
            want.index("layers.0.moe.experts.2.down_proj.weight")
    assert want[-1] == "tok_embeddings.weight"
