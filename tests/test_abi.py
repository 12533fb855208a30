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


def _header_structs(header):
    """Field names of each `typedef struct name { ... } name;` in the header."""
    out = {}
    for m in re.finditer(r"typedef struct (cih_[a-z_]+) \{(.*?)\} \1;", header, re.S):
        body = re.sub(r"/\*.*?\*/", "", m.group(2), flags=re.S)
        names = []
        for decl in body.split(";"):
            decl = decl.strip()
            if decl:
                names += [re.sub(r"[^a-z0-9_]", "", p.split()[-1]) for p in decl.split(",")]
        out[m.group(1)] = names
    return out


def test_integration_extern_block_matches_header():
    """INTEGRATION.md section 1 shows the extern block a maintainer adds to the
    crate: every function it declares exists in include/codon_hip.h with the
    same number of parameters, and its #[repr(C)] structs list the header's
    fields in the header's order (config, host weights, outputs)."""
    with open(os.path.join(REPO, "include", "codon_hip.h")) as f:
        header = f.read()
    with open(os.path.join(REPO, "INTEGRATION.md")) as f:
        doc = f.read()
    sec = doc[doc.index("## 1."):doc.index("## 2.")]
    block = sec[sec.index("```rust"):sec.index("```", sec.index("```rust") + 7)]
    c_funcs = {m.group(1): len([a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"])
               for m in re.finditer(r"\b(?:int|const char \*)\s*(cih_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", header)}
    r_funcs = {m.group(1): len([a for a in m.group(2).split(",") if a.strip()])
               for m in re.finditer(r"pub fn (cih_[a-z0-9_]+)\(([^)]*)\)", block)}
    assert r_funcs, "no declarations found in INTEGRATION.md section 1"
    bad = {k: (c_funcs.get(k), v) for k, v in r_funcs.items() if c_funcs.get(k) != v}
    assert not bad, bad
    structs = _header_structs(header)
    for rust_name, c_name in (("CihConfig", "cih_config"), ("CihHostWeights", "cih_host_weights"),
                              ("CihOutputs", "cih_outputs")):
        m = re.search(r"pub struct " + rust_name + r"\s*\{(.*?)\}", block, re.S)
        assert m, rust_name
        fields = re.findall(r"pub ([a-z0-9_]+)\s*:", m.group(1))
        assert fields == structs[c_name], (rust_name, fields, structs[c_name])


# Exact file sizes of the five presets with the full LM head (reference
# README.md:372-374): FP32 grouped_canonical_v1 (headerless), Q8_0 and Q4_0
# with the 64-byte CODQ header.
PRESET_BYTES = {
    "8M": (30_091_652, 8_864_556, 5_208_516),
    "35M": (134_067_972, 38_636_896, 22_093_636),
    "150M": (592_642_692, 168_646_036, 94_978_756),
    "650M": (2_604_339_332, 738_899_556, 414_617_796),
    "3B": (11_356_354_692, 3_216_540_676, 1_801_205_956),
}
# sequential_hf FP32 sizes the reference detects by length (lib.rs:228-234)
SEQUENTIAL_HF_BYTES = {"8M": 30_092_168, "35M": 134_068_984, "150M": 592_645_160, "650M": 2_604_342_104,
                       "3B": 11_356_360_584}


def _layout_bytes(cfg, dtype):
    """Bytes of a file written in EsmWeights* field order (the loader's and
    save_codq's layout): the layer matrices as 36/20-byte blocks per 32
    weights (FP32: 4 bytes per weight); the token embedding as Q8_0 blocks in
    a Q8_0 file and FP32 otherwise (quantize_q8 / quantize_q4, lib.rs:559-607);
    every vector and the LM head in FP32; plus the CODQ header for quantized
    files."""
    d, F, L, V = cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.vocab_size
    matrices = L * (4 * d * d + 2 * d * F)
    vectors = L * (9 * d + F) + 2 * d + cfg.lm_head_floats()
    per32 = {0: 128, 1: 36, 2: 20}[dtype]
    emb = V * d // 32 * 36 if dtype == 1 else 4 * V * d
    return (64 if dtype else 0) + matrices // 32 * per32 + emb + 4 * vectors


@pytest.mark.parametrize("arch", list(PRESET_BYTES))
def test_preset_file_sizes_and_length_detection(arch, tmp_path):
    """Every preset and format: the layout's total is the reference's
    published file size; a file of exactly that size (header + sparse body)
    passes every format check of cih_model_create_from_file (without a GPU
    the first failure is then the device, CIH_ERR_HIP), and a headerless FP32
    file of the grouped_canonical_v1 or sequential_hf size is recognised by
    its length alone (EsmConfig::detect_from_file_len, lib.rs:195-273),
    while 4 bytes more are not."""
    cfg = ch.EsmConfig.by_name(arch)
    fp32, q8, q4 = PRESET_BYTES[arch]
    assert _layout_bytes(cfg, 0) == fp32 == cfg.grouped_canonical_floats() * 4
    assert _layout_bytes(cfg, 1) == q8 and _layout_bytes(cfg, 2) == q4
    hd = cfg.dim // cfg.n_heads
    assert fp32 + 4 * (hd // 2 + cfg.n_layers * cfg.n_heads + 1) == SEQUENTIAL_HF_BYTES[arch]
    if os.environ.get("CIH_EXPECT_GPU") == "1":
        pytest.skip("with a GPU these files would be loaded in full")
    arch_id = ch.model.ARCH_IDS[arch]

    def sparse(name, size, header=None):
        p = str(tmp_path / name)
        with open(p, "wb") as f:
            if header:
                f.write(header)
            f.truncate(size)
        return p

    for dtype, size in ((1, q8), (2, q4)):
        hdr = _codq_header(dtype, arch_id, cfg)
        assert _create_from_file(sparse(f"{arch}.{dtype}", size, hdr)) == -5, C.lib().cih_last_error()
        assert _create_from_file(sparse(f"{arch}.{dtype}.odd", size - 1, hdr)) == -7      # unaligned classifier
        assert _create_from_file(sparse(f"{arch}.{dtype}.short", 4096, hdr)) == -6        # body cut short
    for name, size in (("grouped", fp32), ("sequential", SEQUENTIAL_HF_BYTES[arch])):
        assert _create_from_file(sparse(f"{arch}.{name}", size)) == -5, C.lib().cih_last_error()
    assert _create_from_file(sparse(f"{arch}.plus4", fp32 + 4)) == -7
    assert b"unrecognized" in C.lib().cih_last_error()
