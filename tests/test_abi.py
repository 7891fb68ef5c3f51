"""The C ABI on the CPU: the library loads, exports every symbol include/qa.h
declares, validates descriptors synchronously (the size guards of
src/decoder.rs:927-950 and src/audio_encoder_gpu.rs:216-245) and reports a
typed error with a message when no device is present (the reference's
device-loss / no-adapter paths, src/gpu.rs:114-126, src/decoder.rs:1670-1672).
No compute call is made here."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header: str, prefix: str) -> set[str]:
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(rf"\b({prefix}_[a-z0-9_]+)\s*\(", text))


def test_exports_every_declared_symbol(pkg):
    declared = _declared(os.path.join(ROOT, "include", "qa.h"), "qa")
    assert declared == set(pkg.EXPORTS), declared ^ set(pkg.EXPORTS)
    lib = ctypes.CDLL(pkg.LIB_PATH)
    for name in declared:
        assert hasattr(lib, name), name


def test_host_mirror_exports(pkg):
    declared = _declared(os.path.join(pkg.CSRC, "host", "qa_host.h"), "qah")
    lib = pkg.host_lib()
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    assert len(declared) >= 20


def test_version(pkg):
    v = pkg.version()
    assert "abi 2" in v and "gfx950" in v


def _desc(pkg, **kw):
    base = dict(dtype=pkg.F16, flags=0, m=64, n=128, k=256, lda=256, ldb=256, ldc=128,
                a=0x100000, w=0x200000, c=0x300000, bias=None, batch=1, bsa=0, bsb=0, bsc=0)
    base.update(kw)
    return pkg.LinearDesc(**base)


def test_validate_accepts_the_reference_shapes(pkg):
    # decoder qkv, o (+res), gu (SiLU), down (+res) at M=1024 (src/decoder.rs:1321-1657)
    big = 1 << 30
    for m, n, k, fl in ((1024, 4096, 1024, 0), (1024, 1024, 2048, pkg.ACCUMULATE),
                        (1024, 6144, 1024, pkg.EPI_SILU_MUL), (1024, 1024, 3072, pkg.ACCUMULATE),
                        (3750, 3584, 896, pkg.EPI_GELU), (3750, 2688, 896, 0)):
        nout = n // 2 if fl & pkg.EPI_SILU_MUL else n
        d = _desc(pkg, m=m, n=n, k=k, lda=k, ldb=k, ldc=nout, flags=fl, a=big, w=2 * big, c=3 * big)
        assert pkg.validate(d) == pkg.QA_OK, pkg.last_error()


@pytest.mark.parametrize("field,value,needle", [
    ("dtype", 7, "dtype"),
    ("flags", 1 << 9, "unknown flags"),
    ("k", 250, "multiple of 8"),
    ("lda", 200, "lda"),
    ("ldb", 100, "ldb"),
    ("ldc", 64, "ldc"),
    ("n", 126, "multiple of 4"),
    ("m", -1, "bad shape"),
    ("a", None, "null operand"),
    ("a", 0x100008, "16-byte aligned"),
    ("c", 0x200000 + 64, "overlaps"),
])
def test_validate_rejects(pkg, field, value, needle):
    d = _desc(pkg, **{field: value})
    rc = pkg.validate(d)
    assert rc == pkg.QA_EINVAL
    assert needle in pkg.last_error(), pkg.last_error()


def test_validate_rejects_epilogue_combinations(pkg):
    bad = [
        dict(flags=pkg.EPI_GELU | pkg.ACCUMULATE),
        dict(flags=pkg.EPI_SILU_MUL, bias=0x400000, ldc=64),
        dict(flags=pkg.EPI_SILU_MUL | pkg.TRANSB, ldc=64),
        dict(flags=pkg.BIAS_ROWS),
        dict(flags=pkg.TRANSB, n=124, ldb=256, ldc=124),
    ]
    for kw in bad:
        assert pkg.validate(_desc(pkg, **kw)) == pkg.QA_EINVAL, kw


def test_calls_without_context_fail_cleanly(pkg):
    lib = pkg.lib()
    d = _desc(pkg)
    assert lib.qa_linear(None, ctypes.byref(d)) == pkg.QA_EINVAL
    assert "null context" in pkg.last_error()
    p = ctypes.c_void_p()
    assert lib.qa_alloc(None, 16, ctypes.byref(p)) == pkg.QA_EINVAL
    assert lib.qa_sync(None) == pkg.QA_EINVAL
    assert lib.qa_ctx_destroy(None) == pkg.QA_OK
    assert lib.qa_ctx_create(0, None) == pkg.QA_EINVAL
    assert lib.qa_prefetch_hint(None, None, 0) == pkg.QA_EINVAL
    assert "null context" in pkg.last_error()
    for fn, desc in ((lib.qa_rms_norm, pkg.RmsNormDesc()), (lib.qa_qk_norm_rope, pkg.QkRopeDesc()),
                     (lib.qa_attention_prefill, pkg.AttentionDesc()),
                     (lib.qa_layer_norm, pkg.LayerNormDesc()),
                     (lib.qa_window_attention, pkg.WindowAttentionDesc()),
                     (lib.qa_add_position_table, pkg.PositionAddDesc()),
                     (lib.qa_conv2d_3x3s2, pkg.ConvDesc()),
                     (lib.qa_log_mel, pkg.MelDesc()),
                     (lib.qa_embed_scatter, pkg.EmbedDesc()),
                     (lib.qa_timestamp_head, pkg.HeadDesc())):
        assert fn(None, ctypes.byref(desc)) == pkg.QA_EINVAL
        assert "null argument" in pkg.last_error()


def test_decoder_descriptor_layouts(pkg):
    """The ctypes mirrors have the C structs' sizes and field offsets (checked
    against a tiny C program compiled from include/qa.h)."""
    import shutil
    import tempfile
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    structs = {"qa_rms_norm_desc": pkg.RmsNormDesc, "qa_qk_rope_desc": pkg.QkRopeDesc,
               "qa_attention_desc": pkg.AttentionDesc, "qa_linear_desc": pkg.LinearDesc,
               "qa_layer_norm_desc": pkg.LayerNormDesc,
               "qa_window_attention_desc": pkg.WindowAttentionDesc,
               "qa_position_add_desc": pkg.PositionAddDesc, "qa_conv_desc": pkg.ConvDesc,
               "qa_mel_desc": pkg.MelDesc, "qa_embed_desc": pkg.EmbedDesc,
               "qa_head_desc": pkg.HeadDesc,
               "qa_mlp_desc": pkg.MlpDesc}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "qa.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as td:
        src, exe = os.path.join(td, "l.c"), os.path.join(td, "l")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), src, "-o", exe], check=True)
        got = dict(l.split() for l in subprocess.run([exe], capture_output=True, text=True,
                                                     check=True).stdout.splitlines())
    for cname, py in structs.items():
        assert int(got[cname]) == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(py, fname).offset, (cname, fname)


def test_no_device_is_a_typed_error():
    """With every device hidden, qa_ctx_create reports QA_EDEVICE and a message
    (run in a child process so the hiding cannot leak into other tests)."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import __graft_entry__ as e\n"
        "pkg = e.load_package()\n"
        "try:\n"
        "    pkg.Context(0)\n"
        "    print('UNEXPECTED')\n"
        "except pkg.QAError as ex:\n"
        "    print(ex.code, ex.message)\n" % ROOT
    )
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    line = out.stdout.strip().splitlines()[-1]
    assert line.startswith(str(-3)), line
    assert "no HIP device" in line


def test_errors_are_thread_local(pkg):
    import threading

    pkg.validate(_desc(pkg, k=250))
    main_msg = pkg.last_error()
    seen = {}

    def worker():
        pkg.validate(_desc(pkg, dtype=9))
        seen["msg"] = pkg.last_error()

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert "dtype" in seen["msg"]
    assert pkg.last_error() == main_msg


def test_mel_filterbank_is_the_oracle_restatement(pkg, orc):
    """qa_mel_filterbank (a host function of the C ABI) and the oracle's
    restatement of create_mel_filterbank agree bit for bit."""
    import numpy as np
    assert np.array_equal(pkg.mel_filterbank(128, 400, 16000), orc.mel_filterbank(128, 400, 16000))
    assert pkg.lib().qa_mel_filterbank(0, 400, 16000, None) == pkg.QA_EINVAL


def test_rope_tables_match_the_text_position_definition(pkg):
    """qa_rope_tables (host) equals the closed form angle = p / theta^(2j/hd)
    with repeated halves (src/mrope.rs:55-89 for text positions)."""
    import numpy as np
    from conftest import rope_tables
    for dt in (pkg.F16, pkg.BF16):
        c, s = pkg.rope_tables(300, 128, 1e6, dt)
        wc, ws = rope_tables(300, 128, 0, theta=1e6, dtype=dt)
        assert np.array_equal(c, wc) and np.array_equal(s, ws)
    # every value is a 16-bit value widened: the reference narrows both tables
    # (src/align_inference.rs:371-372, 394-395)
    c, s = pkg.rope_tables(300, 128, 1e6, pkg.F16)
    assert np.array_equal(c, c.astype(np.float16).astype(np.float32))
    c, s = pkg.rope_tables(300, 128, 1e6, pkg.BF16)
    assert not (c.view(np.uint32) & 0xFFFF).any() and not (s.view(np.uint32) & 0xFFFF).any()
    assert pkg.lib().qa_rope_tables(4, 128, 1e6, 7, c.ctypes.data, s.ctypes.data) == pkg.QA_EINVAL
