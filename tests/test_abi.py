"""CPU checks of the C ABI: the library loads, exports every symbol the header
declares with the binding's signature table, and its host-only entry points
(workspace sizing, the reference Rng) behave.  No kernel is launched here."""
import ctypes as C
import re

import numpy as np
import pytest

from conftest import ROOT


def _header_symbols():
    text = (ROOT / "include" / "asca_hip.h").read_text()
    return sorted(set(re.findall(r"ASCA_API\s+[\w\s\*]+?\b(asca_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from asca_amd import _lib

    lib = _lib.load()
    names = _header_symbols()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} missing from the ctypes signature table"
    assert set(_lib.SIGNATURES) == set(names)


_C2RUST = {"int": "c_int", "long": "i64", "size_t": "usize", "float": "f32", "uint32_t": "u32", "uint64_t": "u64",
           "int64_t": "i64", "int32_t": "i32", "uint16_t": "u16", "char": "c_char", "void": "c_void",
           "asca_model": "AscaModel"}


def _rust_type(c_type: str) -> str:
    """The Rust FFI spelling of a C parameter / return type (sys.rs style)."""
    t = c_type.strip()
    const = t.startswith("const ")
    if const:
        t = t[len("const "):]
    stars = t.count("*")
    r = _C2RUST[t.replace("*", "").strip()]
    if stars:
        r = ("*const " if const else "*mut ") + r
        r = "*mut " * (stars - 1) + r
    return r


def _header_prototypes():
    text = (ROOT / "include" / "asca_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    out = {}
    for m in re.finditer(r"ASCA_API\s+([\w\s\*]+?)\b(asca_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, params = " ".join(m.group(1).split()), m.group(3).strip()
        types = []
        for p in ([] if params in ("", "void") else params.split(",")):
            p = " ".join(p.split())
            types.append(_rust_type(p[: -len(re.search(r"(\w+)$", p).group(1))].replace(" *", "*")))
        out[m.group(2)] = (types, "" if ret == "void" else _rust_type(ret))
    return out


def _integration_externs():
    text = (ROOT / "INTEGRATION.md").read_text()
    out = {}
    for m in re.finditer(r"pub fn (asca_\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", text):
        types = [" ".join(p.split(":", 1)[1].split()) for p in m.group(2).split(",") if p.strip()]
        out[m.group(1)] = (types, (m.group(3) or "").strip())
    return out


def test_integration_extern_blocks_match_the_header():
    """The Rust extern blocks a maintainer pastes into the reference crate
    (rust/src/hip/sys.rs, replacing rust/src/cuda/sys.rs) declare every entry
    point of the header, each with the header's parameter and return types."""
    hdr, rs = _header_prototypes(), _integration_externs()
    assert set(hdr) == set(_header_symbols())
    assert sorted(set(hdr) - set(rs)) == [], "entry points missing from INTEGRATION.md"
    assert sorted(set(rs) - set(hdr)) == [], "INTEGRATION.md declares entry points the header lacks"
    for name, proto in hdr.items():
        assert rs[name] == proto, name


def test_workspace_bytes_layout():
    from asca_amd import _lib

    out = C.c_size_t()
    _lib.call("asca_delta_ws_bytes", 32, 512, 8, 64, C.byref(out))
    sk = 32 * 512 * 8 * 64 * 4
    # dh = 64 on a block per unit (the blocked form): the u rows (per unit and
    # 16-step block, T rounded up to whole blocks), a checkpoint before every
    # other 16-step block plus the state after the last step, and a 1344-float
    # record per block (K K^T, Q K^T, T, M, Gamma, the gate vectors); the
    # backward writes nothing into it
    ckpt = 32 * 8 * (512 // 32 + 1) * 64 * 64 * 4
    rec = 32 * 8 * (512 // 16) * 1344 * 4
    assert out.value == sk + ckpt + rec
    # at most 128 (sequence, head) units: each unit's columns run on two blocks;
    # their partial dq, dk and dalpha, dbeta live in the backward call's own
    # scratch, not in the forward's workspace
    _lib.call("asca_delta_ws_bytes", 4, 128, 4, 32, C.byref(out))
    base = 4 * 128 * 4 * 32 * 4 + 4 * 4 * (128 // 8 + 1) * 32 * 32 * 4
    assert out.value == base
    # dh = 64 runs a block per unit at any unit count (configs[3]'s 128 units too)
    _lib.call("asca_delta_ws_bytes", 16, 1024, 8, 64, C.byref(out))
    assert out.value == (16 * 1024 * 8 * 64 * 4 + 16 * 8 * (1024 // 32 + 1) * 64 * 64 * 4
                         + 16 * 8 * (1024 // 16) * 1344 * 4)
    _lib.call("asca_delta_ws_bytes", 1, 40, 2, 64, C.byref(out))
    assert out.value == (256 * ((1 * 48 * 2 * 64 * 4 + 255) // 256) + 2 * (40 // 32 + 2) * 64 * 64 * 4
                         + 256 * ((2 * 3 * 1344 * 4 + 255) // 256))
    with pytest.raises(_lib.AscaError) as ei:
        _lib.call("asca_delta_ws_bytes", 1, 1, 1, 129, C.byref(out))
    assert ei.value.code == 3


def test_product_rng_equals_oracle_rng(orc):
    from asca_amd import _lib

    lib = _lib.load()
    st = (C.c_uint64 * 2)()
    for seed in range(4):
        lib.asca_rng_seed(seed, st)
        out = np.zeros(16, dtype=np.uint64)
        lib.asca_rng_u64(st, out.ctypes.data_as(C.POINTER(C.c_uint64)), 16)
        np.testing.assert_array_equal(out, orc.rng_u64(seed, 16))
    lib.asca_rng_seed(1, st)
    got = np.zeros(1000, dtype=np.float32)
    lib.asca_rng_normal(st, got.ctypes.data_as(C.c_void_p), 1000, 1.0, 0.0)
    np.testing.assert_array_equal(got, orc.rng_normal(1, 1000))


def test_errors_without_device_are_codes_not_aborts():
    from asca_amd import _lib

    lib = _lib.load()
    n = C.c_int(0)
    if lib.asca_device_count(C.byref(n)) == 0 and n.value > 0:
        pytest.skip("a GPU is present; this checks the no-device path")
    rc = lib.asca_init(0)
    assert rc != 0
    assert lib.asca_last_error()
    # entry points fail cleanly before init (no HIP call is reached)
    fake = C.c_void_p(0x1000)
    rc = lib.asca_delta_fwd(fake, fake, fake, fake, fake, fake, fake, 1, 4, 1, 16, None)
    assert rc == 4
