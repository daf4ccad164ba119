"""The C-ABI boundary and the host-side mirror, without a GPU.

Checks that libredukt_gpu.so loads and exports every symbol include/redukt_backend.h
declares, that the struct layout and result codes are the reference's, that the
pre-init error paths answer without touching a device, and the host logic
(validate_batch_args, .rbin header parsing, slot pool) against the reference's own test
cases held in tests/golden/reference_known_answers.json.
"""
import ctypes
import json
import os
import re
import struct

import numpy as np
import pytest

from redukt_amd import LIB_PATH, ffi, rbin

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_known_answers.json")))
HEADER = os.path.join(ROOT, "include", "redukt_backend.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(redukt_backend_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def raw_lib():
    if not os.path.isfile(LIB_PATH):
        pytest.fail(f"{LIB_PATH} not built: run __graft_entry__.build()")
    return ctypes.CDLL(LIB_PATH)


def test_header_declares_reference_symbols():
    syms = declared_symbols()
    for s in ffi.V1_SYMBOLS + ffi.V2_SYMBOLS + ffi.V3_SYMBOLS:
        assert s in syms, s
    assert len(syms) == len(ffi.V1_SYMBOLS + ffi.V2_SYMBOLS + ffi.V3_SYMBOLS)


def test_profile_bits_match_the_header():
    """Every weight-profile bit the header defines has the same value in the Python mirror,
    and the oracle's profile constants agree with both."""
    from oracle import oracle as O

    text = open(HEADER).read()
    defs = {k: int(v) for k, v in re.findall(r"#define BACKEND_PROFILE_(\w+) (\d+)u", text)}
    assert len(defs) == 9
    for name, value in defs.items():
        assert getattr(ffi, "PROFILE_" + name) == value, name
    for name in ("EXACT", "FMA"):
        assert getattr(O, "ORC_PROFILE_" + name) == defs[name], name
    orc = dict(re.findall(r"ORC_PROFILE_(\w+) = (\d+)", open(os.path.join(ROOT, "oracle", "oracle.h")).read()))
    for name in ("F32", "Q8_G64", "Q8_ROW", "Q8_SMALL", "W8A8", "EXACT", "FMA"):
        assert int(orc[name]) == defs[name], name


def test_library_exports_every_declared_symbol(raw_lib):
    for s in declared_symbols():
        assert hasattr(raw_lib, s), f"missing export {s}"


def test_backend_info_layout():
    assert ctypes.sizeof(ffi.BackendInfo) == 76
    assert ffi.BackendInfo.name.offset == 12
    info = ffi.BackendInfo()
    label = b"wgpu-vulkan"
    for i, b in enumerate(label):
        info.name[i] = b
    assert info.name_str() == "wgpu-vulkan"
    assert ffi.BackendInfo().name_str() == ""


def test_result_codes_and_from_code():
    g = GOLD["backend_result_codes"]
    for name, code in g["codes"].items():
        assert int(ffi.BackendResult[name]) == code
        assert ffi.BackendResult.from_code(code) == ffi.BackendResult[name]
    for code, name in g["from_code_unknown"]:
        assert ffi.BackendResult.from_code(code) == ffi.BackendResult[name]


def test_validate_batch_args_reference_cases():
    g = GOLD["validate_batch_args"]
    for c in g["accept"]:
        seen = [False] * c["seen_len"]
        assert ffi.validate_batch_args(c["slots"], c["tokens"], c["out_len"], c["vocab"], c["max_streams"], seen) is None
    for c in g["reject"]:
        seen = [False] * c["seen_len"]
        r = ffi.validate_batch_args(c["slots"], c["tokens"], c["out_len"], c["vocab"], c["max_streams"], seen)
        assert r == ffi.BackendResult.INVALID_ARGUMENT, c["why"]


def test_rbin_header_reference_cases():
    g = GOLD["rbin_header"]

    def header(version, vocab, word10):
        return struct.pack("<11I", rbin.RBIN_MAGIC, version, vocab, *g["header_words_tail"], word10)

    for c in g["parse"]:
        got = rbin.parse_rbin_header(header(c["version"], c["vocab"], c["word10"]))
        if c["expect"] is None:
            assert got is None
        else:
            assert got == rbin.RbinMeta(c["expect"]["version"], c["expect"]["vocab_size"], c["expect"]["tokenizer"])
    assert rbin.parse_rbin_header(header(1, 256, 0)[:40]) is None
    bad = bytearray(header(1, 256, 0))
    bad[0] ^= 0xFF
    assert rbin.parse_rbin_header(bytes(bad)) is None
    for src, want in g["path_rule"]:
        assert rbin.rbin_path(src) == os.path.join(*want.split("/"))


def test_rbin_writer_round_trip(tmp_path):
    dims = rbin.MambaDims(vocab=300, d_model=32, n_layer=2)
    from redukt_amd import synth
    p = str(tmp_path / "m.rbin")
    synth.write_synthetic_mamba(p, dims, seed=1, flags=rbin.FLAG_NORM_BIAS | rbin.FLAG_UNTIED_HEAD)
    d2, flags, t = rbin.read_rbin(p)
    assert d2 == dims and flags == 3
    assert set(t) == {n for n, _ in rbin.tensor_order(dims, flags)}
    meta = rbin.parse_rbin_header(open(p, "rb").read(44))
    assert meta == rbin.RbinMeta(2, 300, rbin.TOK_BPE)
    expected_floats = sum(int(np.prod(s)) for _, s in rbin.tensor_order(dims, flags))
    assert os.path.getsize(p) == 44 + 4 * expected_floats


def test_mamba_130m_weight_bytes():
    # Weight bytes streamed per token (published: 516.5 MB F32, 153.6 MB Q8 groups of 64).
    d = rbin.MAMBA_130M
    V, dm, di, ds, dc, dr, L = d.vocab, d.d_model, d.d_inner, d.d_state, d.d_conv, d.dt_rank, d.n_layer
    small = dm + di * dc + di + (dr + 2 * ds) * di + di * dr + di + di * ds + di
    big = 2 * di * dm + dm * di
    f32 = 4 * (L * (small + big) + dm + V * dm)
    q8_g64 = 4 * (L * small + dm) + L * (big + big // 64 * 4) + V * dm + V * dm // 64 * 4
    assert f32 == 516_541_440
    assert q8_g64 == 153_614_208


def test_slot_pool_reference_case():
    p = ffi.SlotPool()
    assert p.take() is None
    p.init(3)
    assert [p.take() for _ in range(4)] == GOLD["slot_pool"]["init3_takes"]
    assert len(p.seen) == 3
    p.init(1)
    assert [p.take() for _ in range(2)] == GOLD["slot_pool"]["reinit1_takes"]


def test_pre_init_error_paths_touch_no_device():
    lib = ffi.PluginLibrary(LIB_PATH)
    L = lib.lib
    assert lib.abi_version == ffi.BACKEND_ABI_V3 and lib.has_v3
    out = np.zeros(4, np.float32)
    s = np.zeros(1, np.uint32)
    p32 = lambda a, t: a.ctypes.data_as(ctypes.POINTER(t))
    assert L.redukt_backend_forward(0, p32(out, ctypes.c_float), 4) == ffi.BackendResult.FORWARD_FAILED
    assert L.redukt_backend_batch_init(4) == ffi.BackendResult.INIT_FAILED
    assert L.redukt_backend_batch_reset(None, 0) == ffi.BackendResult.INIT_FAILED
    assert L.redukt_backend_forward_batch(1, p32(s, ctypes.c_uint32), p32(s, ctypes.c_uint32),
                                          p32(out, ctypes.c_float), 4) == ffi.BackendResult.INIT_FAILED
    assert L.redukt_backend_forward_batch_probs(1, p32(s, ctypes.c_uint32), p32(s, ctypes.c_uint32),
                                                p32(out, ctypes.c_float), 4) == ffi.BackendResult.INIT_FAILED
    assert L.redukt_backend_forward_batch_device(1, None, None, None, 4, 0) == ffi.BackendResult.INIT_FAILED
    assert L.redukt_backend_device_status() == ffi.BackendResult.INIT_FAILED
    assert L.redukt_backend_get_state(0, 0, None, None) == ffi.BackendResult.INIT_FAILED
    assert L.redukt_backend_stream() is None
    # the measurement copy validates its arguments before anything reaches the GPU
    assert L.redukt_backend_copy_probe(None, None, 0, 0) == ffi.BackendResult.OK
    for dst, src, nbytes, mode in ((None, None, 16, 0), (1, 1, 15, 0), (1, 1, 16, 4), (1, 1, 1 << 31, 1)):
        assert L.redukt_backend_copy_probe(dst, src, nbytes, mode) == ffi.BackendResult.INVALID_ARGUMENT
    info = ffi.BackendInfo()
    assert L.redukt_backend_init(None, 0, ctypes.byref(info)) == ffi.BackendResult.INIT_FAILED
    # bits 0-7 are defined (quant, small-matrix quant, exact scan, GEMV tier, RWKV-7 W8A8,
    # the reference-order tier and its contract 2); anything above is refused
    assert L.redukt_backend_init_ex(b"x.rbin", 0, 256, ctypes.byref(info)) == ffi.BackendResult.INVALID_ARGUMENT
    L.redukt_backend_reset_state()   # no model: a no-op
    L.redukt_backend_free()          # idempotent


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(FileNotFoundError):
        ffi.PluginLibrary(str(tmp_path / "libredukt_gpu.so"))
