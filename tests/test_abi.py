"""The C-ABI library loads and exports every entry point declared in include/*.h.

No computation runs here (this suite also runs where there is no GPU); the
host-only table builder is checked against the oracle, and without a GPU the
library reports SMOL_ATTN_ERR_NO_GPU instead of computing anything on the CPU.
"""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT, pkg  # noqa: F401

INCLUDE = os.path.join(ROOT, "include")
DECL = re.compile(r"SMOL_(?:ATTN|KERNELS)_API\s+[\w\s\*]*?\b(\w+)\s*\(", re.S)


def declared():
    names = []
    for f in sorted(os.listdir(INCLUDE)):
        if f.endswith(".h"):
            with open(os.path.join(INCLUDE, f)) as fh:
                text = "\n".join(l for l in fh.read().splitlines() if not l.lstrip().startswith("#"))
                names += DECL.findall(text)
    return names


def test_library_exports_every_declared_symbol():
    from smol_genius_amd import smol_attn as sa
    lib = sa.load()
    names = declared()
    assert len(names) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", sa.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        assert getattr(lib, n) is not None
    # the Python mirror binds exactly the declared set
    assert sorted(n for n, _, _ in sa.SIGNATURES) == sorted(names)
    # nothing else leaks out of the library with default visibility
    extra = sorted(e for e in exported if e.startswith("smol_") and e not in names)
    assert not extra, extra


def test_version_string():
    from smol_genius_amd import smol_attn as sa
    assert b"gfx950" in sa.load().smol_attn_version()


def test_host_rope_table_matches_oracle(oracle):
    from smol_genius_amd import smol_attn as sa
    for hd, theta, rt in [(128, 1e6, 0), (256, 1e4, 1), (72, 1e4, 0), (64, 1e6, 1)]:
        c, s = sa.rope_fill_host(0, 8300, hd, theta, rt)
        oc, os_ = oracle.fill_rope_table(0, 8300, hd, theta, rt == 1)
        np.testing.assert_array_equal(c, oc)
        np.testing.assert_array_equal(s, os_)
        c2, s2 = sa.rope_fill_host(4000, 5, hd, theta, rt)
        np.testing.assert_array_equal(c2, oc[4000:4005])


def test_no_gpu_means_no_compute():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from smol_genius_amd import smol_attn as sa
    lib = sa.load()
    assert lib.smol_attn_device_count() == -5
    h = ctypes.c_void_p()
    assert lib.smol_attn_ctx_create(0, None, ctypes.byref(h)) == -5
    assert b"no HIP device" in lib.smol_attn_last_error()
    with pytest.raises(sa.SmolAttnError):
        sa.Context(0, stream=0)


LLVM_BIN = "/opt/rocm/llvm/bin"


def _gfx950_disassembly(tmp_path):
    """Disassembly of the gfx950 code objects embedded in the built library (the
    .hip_fatbin section holds one offload bundle per translation unit)."""
    from smol_genius_amd import smol_attn as sa
    tools = [os.path.join(LLVM_BIN, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")]
    if not all(os.path.exists(t) for t in tools):
        pytest.skip("ROCm LLVM tools not present")
    objcopy, bundler, objdump = tools
    fb = str(tmp_path / "fatbin.bin")
    subprocess.run([objcopy, "--dump-section", ".hip_fatbin=" + fb, sa.LIB_PATH, str(tmp_path / "x.so")],
                   check=True, capture_output=True)
    data = open(fb, "rb").read()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts = [i for i in range(len(data)) if data.startswith(magic, i)] if magic in data else []
    assert starts, "no offload bundle in the library"
    lines = []
    for n, a in enumerate(starts):
        b = starts[n + 1] if n + 1 < len(starts) else len(data)
        part, co = str(tmp_path / ("b%d.bin" % n)), str(tmp_path / ("b%d.co" % n))
        open(part, "wb").write(data[a:b])
        subprocess.run([bundler, "--type=o", "--unbundle", "--input=" + part, "--output=" + co,
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950"], check=True, capture_output=True)
        out = subprocess.run([objdump, "-d", "--mcpu=gfx950", co], check=True, capture_output=True,
                             text=True).stdout
        lines += [l.split("//")[0].strip() for l in out.splitlines() if l.startswith("\t") or l.startswith(" ")]
    return lines


def test_m0_only_written_for_lds_transfers(tmp_path):
    """Every instruction of the library's gfx950 code that names M0 is the LDS-DMA sequence
    s_mov_b32 m0, sN / s_nop 0 / buffer_load_dwordx4 ... lds (one wait state between the M0
    write and the transfer that reads it), and every LDS transfer is preceded by it. The
    kernels' transfers are inline asm, invisible to the compiler's hazard recognizer, so this
    checks the built code rather than the source."""
    ins = [l for l in _gfx950_disassembly(tmp_path) if l]
    n_dma = 0
    for i, l in enumerate(ins):
        if re.search(r"\bm0\b", l):
            assert re.fullmatch(r"s_mov_b32 m0, s\d+", l), l
            assert ins[i + 1] == "s_nop 0", (l, ins[i + 1])
            assert ins[i + 2].startswith("buffer_load_dwordx4") and ins[i + 2].endswith(" lds"), ins[i + 2]
        if l.startswith("buffer_load") and l.endswith(" lds"):
            n_dma += 1
            assert ins[i - 1] == "s_nop 0" and ins[i - 2].startswith("s_mov_b32 m0,"), (ins[i - 2], ins[i - 1], l)
    assert n_dma > 0


def test_decoder_block_argument_errors_without_device_work():
    """The decoder-level block rejects an unbound owner and a bad config
    before any device call; unbinding an unknown owner is not an error."""
    from smol_genius_amd import smol_attn as sa
    lib = sa.load()
    owner = ctypes.create_string_buffer(64)
    addr = ctypes.c_void_p(ctypes.addressof(owner))
    assert lib.smol_qkn_attn_prefill(addr, 0, 0, 1, None, None, None, None) == -1
    assert b"not bound" in lib.smol_attn_last_error()
    assert lib.smol_qkn_attn_forward(addr, 0, 0, None, None, None, None) == -1
    assert lib.smol_qkn_attn_set_layer(addr, 0, 0, None, None) == -1
    assert lib.smol_qkn_attn_unbind(addr) == 0
    bad = sa.QknConfig(n_layers=2, n_heads=6, n_kv_heads=4, head_dim=128, eps=1e-6, rope_theta=1e6,
                       rope_type=0, max_seq=64)   # 6 heads over 4 KV heads
    assert lib.smol_qkn_attn_bind(addr, ctypes.byref(bad)) == -1
    bad.n_kv_heads, bad.head_dim = 2, 100     # unsupported head_dim
    assert lib.smol_qkn_attn_bind(addr, ctypes.byref(bad)) == -1
    bad.head_dim = 128
    rc = lib.smol_qkn_attn_bind(addr, ctypes.byref(bad))
    if rc == 0:   # a GPU is present
        assert lib.smol_qkn_attn_unbind(addr) == 0
    else:
        assert rc == -5   # SMOL_ATTN_ERR_NO_GPU


REF_KERNELS_H = "/root/reference/common/kernels/smol_kernels.h"


@pytest.mark.skipif(not os.path.exists(REF_KERNELS_H), reason="reference tree not present")
def test_drop_in_header_agrees_with_reference_header(tmp_path):
    """include/smol_kernels_attn.h and the reference's smol_kernels.h in one
    C translation unit (the reference header is C only: it has no extern "C"
    block): a prototype that differs in any parameter or return type is a
    conflicting redeclaration, which the compiler rejects."""
    cc, std = "gcc", "-std=c11"
    src = tmp_path / "tu.c"
    src.write_text('#include "%s"\n#include "smol_kernels_attn.h"\n#include "smol_kernels_linear.h"\n'
                   '#include "smol_qkn_attn.h"\n#include "smol_linear.h"\nint main(void) { return 0; }\n'
                   % REF_KERNELS_H)
    r = subprocess.run([cc, std, "-Wall", "-Werror", "-fsyntax-only", "-I" + INCLUDE, str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # the check bites: a drifted prototype is rejected
    bad = tmp_path / "bad.c"
    bad.write_text('#include "%s"\nvoid smol_causal_attention(float *out, const float *Q, const float *K, '
                   'const float *V, int seq_q, int seq_k, int n_heads, int n_kv_heads, int head_dim, '
                   'double scale, int q_offset);\n' % REF_KERNELS_H)
    r = subprocess.run([cc, std, "-fsyntax-only", str(bad)], capture_output=True, text=True)
    assert r.returncode != 0


@pytest.mark.parametrize("hdr", ["smol_attn.h", "smol_kernels_attn.h", "smol_qkn_attn.h", "smol_linear.h",
                                 "smol_kernels_linear.h"])
def test_public_headers_compile_alone_as_c(tmp_path, hdr):
    src = tmp_path / "one.c"
    src.write_text('#include "%s"\n' % hdr)
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", "-fsyntax-only",
                        "-I" + INCLUDE, str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


REF_DECODER = "/root/reference/common/decoder"


def _integration_c_blocks():
    """The ```c code blocks of the integration guide's decoder-level section
    (its second section), in order."""
    import re
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("## 2."):text.index("## 3.")]
    return re.findall(r"```c\n(.*?)```", sec, re.S)


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_DECODER, "qkn_decoder.h")),
                    reason="the reference tree is not present")
def test_integration_snippets_compile_against_reference_decoder(tmp_path):
    """The decoder-level replacement the integration guide shows for
    qkn_decoder.c:460-528 / :625-677 (and the device layer loop) compiles as
    one C11 translation unit against the reference's own qkn_decoder.h and
    this repository's headers: every qkn_ctx_t / qkn_config_t field and every
    library signature it uses is checked. A snippet that names a field the
    reference struct does not have is rejected (the check bites)."""
    blocks = _integration_c_blocks()
    assert len(blocks) >= 3, "the section's code blocks"
    inc = ["-I" + REF_DECODER, "-I" + os.path.join(os.path.dirname(REF_DECODER), "utils"), "-I" + INCLUDE]
    src = tmp_path / "integration.c"
    src.write_text("\n".join(blocks))
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-Wno-unused-function", "-fsyntax-only"]
                       + inc + [str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    bad = tmp_path / "bad.c"
    bad.write_text("\n".join(blocks).replace("ctx->pref_attn_out", "ctx->pref_attention_out"))
    r = subprocess.run(["gcc", "-std=c11", "-fsyntax-only"] + inc + [str(bad)], capture_output=True, text=True)
    assert r.returncode != 0
