"""CPU checks of the C ABI library (no GPU calls that need a device):
symbol exports, the host-side quantizers / tokenizer / log-softmax against
the oracle, argument and file-format error paths, and the CODQ reader."""
import ctypes
import os
import re
import struct

import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from codon_hip import _lib as C
from conftest import REPO


def test_exports_every_declared_symbol():
    with open(os.path.join(REPO, "include", "codon_hip.h")) as f:
        text = f.read()
    declared = sorted(set(re.findall(r"\b(cih_[a-z0-9_]+)\s*\(", text)))
    lib = ctypes.CDLL(C.LIB_PATH)
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(C.EXPORTED) == declared
    assert lib.cih_abi_version() == 1


@pytest.mark.parametrize("dtype", [1, 2])
def test_host_quantizers_bit_exact_vs_oracle(dtype):
    rng = np.random.default_rng(dtype)
    x = np.concatenate([
        rng.standard_normal(32 * 2000).astype(np.float32) * np.float32(0.02),
        rng.standard_normal(32 * 100).astype(np.float32) * np.float32(1e4),
        np.zeros(32, np.float32),
        np.full(32, -7.0, np.float32),
        np.array([np.nan] + [1.0] * 31, np.float32),
        (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5),  # exact halves
    ])
    mine = ch.quantize_slice_to_q8(x) if dtype == 1 else ch.quantize_slice_to_q4(x)
    ref = cr.quantize_q8(x) if dtype == 1 else cr.quantize_q4(x)
    assert np.array_equal(mine, ref)
    fin = np.isfinite(x).reshape(-1, 32).all(1)
    bb = 36 if dtype == 1 else 20
    dq = ch.dequantize_blocks(dtype, mine).reshape(-1, 32)
    dr = (cr.dequantize_q8(ref) if dtype == 1 else cr.dequantize_q4(ref)).reshape(-1, 32)
    assert np.array_equal(dq[fin].view(np.uint32), dr[fin].view(np.uint32))
    assert mine.size == x.size // 32 * bb


def test_tokenizer_and_log_softmax_vs_oracle():
    for s in ["", "LA", "M<mask>C<mask_1>", "ACDEFGHIKLMNPQRSTVWYXBUZO.-*?", "Aé€😀L"]:
        assert np.array_equal(ch.Tokenizer.encode(s), cr.tokenize(s)), s
    x = np.random.default_rng(0).standard_normal(33).astype(np.float32)
    assert np.array_equal(ch.log_softmax_canonical(x), cr.log_softmax_canonical(x))


def test_argument_errors_without_device():
    lib = C.lib()
    out = np.empty(36, np.uint8)
    x = np.zeros(33, np.float32)
    assert lib.cih_quantize_q8(x.ctypes.data, 33, out.ctypes.data) == -1       # not a multiple of 32
    assert lib.cih_tokenize(b"LLLL", out.ctypes.data, 3) == -1                  # capacity
    assert lib.cih_forward(None, None, None, 1, 1, 0, None) == -1
    assert lib.cih_model_reserve(None, 1, 1, 0) == -1
    assert lib.cih_model_destroy(None) == 0
    assert b"null" in lib.cih_last_error()


def _codq_header(dtype, arch_id, cfg):
    """CodqHeader (lib.rs:887-898): magic, version 1, dtype, arch, layers,
    dim, hidden, vocab, 32 zero bytes."""
    return b"CODQ" + struct.pack("<7I", 1, dtype, arch_id, cfg.n_layers, cfg.dim, cfg.hidden_dim,
                                  cfg.vocab_size) + bytes(32)


def write_codq(path, cfg, w, arch_id):
    """EsmWeightsQ8/Q4::save_to_file[_with_header] field order (lib.rs:716-742, 1128-1154)."""
    with open(path, "wb") as f:
        f.write(_codq_header(w.dtype, arch_id, cfg))
        for k in ch.model.FIELDS:
            f.write(np.ascontiguousarray(getattr(w, k)).tobytes())


def _create_from_file(path, quantize_to=-1):
    """Status of cih_model_create_from_file; a model it creates is destroyed."""
    h = ctypes.c_void_p()
    rc = C.lib().cih_model_create_from_file(path.encode(), quantize_to, None, 0.0, ctypes.byref(h))
    if rc == 0:
        assert h.value
        assert C.lib().cih_model_destroy(h) == 0
    return rc


def test_file_reader_errors(tmp_path):
    p = str(tmp_path / "junk.bin")
    with open(p, "wb") as f:
        f.write(b"\0" * 1000)
    assert _create_from_file(p) == -7                                  # CIH_ERR_FORMAT
    assert _create_from_file(str(tmp_path / "missing.bin")) == -6      # CIH_ERR_IO
    cfg = ch.EsmConfig.esm2_8m()
    bad = str(tmp_path / "badver.bin")
    hdr = bytearray(_codq_header(1, 0, cfg))
    hdr[4] = 99                                                        # version 99
    with open(bad, "wb") as f:
        f.write(bytes(hdr) + b"\0" * 64)
    assert _create_from_file(bad) == -7 and b"version" in C.lib().cih_last_error()
    inc = str(tmp_path / "incoherent.bin")
    with open(inc, "wb") as f:
        f.write(_codq_header(1, 0, ch.EsmConfig(999, 1280, 6, 20)) + b"\0" * 64)
    assert _create_from_file(inc) == -7
    short = str(tmp_path / "short.bin")                                # header + truncated body
    with open(short, "wb") as f:
        f.write(_codq_header(1, 0, cfg) + b"\0" * 1000)
    assert _create_from_file(short) == -6


def test_file_reader_accepts_valid_files(tmp_path, w8m_path):
    """Valid inputs parse completely: without a GPU the first failure is the
    device check (CIH_ERR_HIP), after every format check has passed; with a
    GPU (CIH_EXPECT_GPU=1) every load succeeds and its model is destroyed.
    The loads' numbers are checked against the oracle in test_gpu_loader.py."""
    cfg = ch.EsmConfig.esm2_8m()
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)
    q8 = str(tmp_path / "m.q8")
    write_codq(q8, cfg, w.quantize_q8(), 0)
    q4 = str(tmp_path / "m.q4")
    write_codq(q4, cfg, w.quantize_q4(), 0)
    on_gpu = os.environ.get("CIH_EXPECT_GPU") == "1"
    for path, qt in ((w8m_path, -1), (w8m_path, 1), (w8m_path, 2), (q8, -1), (q4, -1)):
        rc = _create_from_file(path, qt)
        assert rc == (0 if on_gpu else -5), (path, qt, C.lib().cih_last_error())
    # a Q8 file cannot be requantized to Q4
    assert _create_from_file(q8, 2) == -1


def test_capi_driver_builds_and_reports_errors(w8m_path):
    """The C caller (capi/pipeline.c) is built with the library; without a
    device it stops at the first HIP call with the library's message."""
    import subprocess
    drv = os.path.join(REPO, "codon-infer_amd", "capi", "pipeline")
    assert os.path.exists(drv)
    r = subprocess.run([drv], capture_output=True, text=True)
    assert r.returncode == 2 and "usage" in r.stderr
    if os.environ.get("CIH_EXPECT_GPU") != "1":
        r = subprocess.run([drv, "dms", w8m_path, "LAGV", "0", "0", "0", "2"], capture_output=True, text=True)
        assert r.returncode == 1 and "cih_model_create_from_file failed (-5)" in r.stderr, r.stderr


def test_rust_ffi_declares_every_entry_point():
    """rust/codon-hip-sys/src/lib.rs declares exactly the functions of
    include/codon_hip.h, with the same number of parameters (no cargo in
    this image, so this is the check that the binding tracks the header)."""
    with open(os.path.join(REPO, "include", "codon_hip.h")) as f:
        header = f.read()
    with open(os.path.join(REPO, "rust", "codon-hip-sys", "src", "lib.rs")) as f:
        rust = f.read()
    c_funcs = {}
    for m in re.finditer(r"\b(?:int|const char \*)\s*(cih_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", header):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        c_funcs[m.group(1)] = len(args)
    r_funcs = {}
    for m in re.finditer(r"pub fn (cih_[a-z0-9_]+)\(([^)]*)\)", rust):
        args = [a for a in m.group(2).split(",") if a.strip()]
        r_funcs[m.group(1)] = len(args)
    assert c_funcs and c_funcs == r_funcs, (set(c_funcs) ^ set(r_funcs),
                                            {k: (c_funcs.get(k), r_funcs.get(k)) for k in c_funcs
                                             if c_funcs.get(k) != r_funcs.get(k)})
