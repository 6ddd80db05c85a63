"""The C ABI without a GPU: the library loads, exports every function that
include/llmk_sampler.h declares, its ctypes mirror has the C layout, and the
argument checks that run before any device call return the documented codes.
Also: the product package never reaches the oracle and fails loudly when the
library is missing."""
import ctypes
import os
import re
import subprocess

import pytest

import llmk
from llmk import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "llmk_sampler.h")


def declared_functions():
    src = open(HDR).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(llmk_[a-z_]+)\s*\(", src)))


def test_header_declarations_are_the_exported_list():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    assert os.path.exists(_lib.LIB_PATH), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    for name in declared_functions():
        assert name in exported, name
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name)


def test_ctypes_struct_matches_c_layout(tmp_path):
    """offsetof/sizeof of llmk_sample_batch_args from the C compiler."""
    fields = [f for f, _ in _lib.SampleBatchArgs._fields_]
    prog = tmp_path / "layout.c"
    body = "".join(f'  printf("{f} %zu\\n", offsetof(llmk_sample_batch_args, {f}));\n' for f in fields)
    prog.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "llmk_sampler.h"\n'
                    "int main(void){\n" + body +
                    '  printf("SIZE %zu\\n", sizeof(llmk_sample_batch_args));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(prog), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                  check=True).stdout.splitlines())
    for f in fields:
        assert int(got[f]) == getattr(_lib.SampleBatchArgs, f).offset, f
    assert int(got["SIZE"]) == ctypes.sizeof(_lib.SampleBatchArgs)


def test_constants_match_header():
    src = open(HDR).read()
    for name in ("LLMK_OK", "LLMK_ERR_INVALID_ARGUMENT", "LLMK_ERR_EMPTY_LOGITS", "LLMK_ERR_CAPACITY",
                 "LLMK_ERR_HIP", "LLMK_ERR_ALIGNMENT", "LLMK_ERR_UNSUPPORTED",
                 "LLMK_STATUS_INVALID_PARAMS", "LLMK_STATUS_HISTORY_OVERFLOW",
                 "LLMK_STATUS_SLOT_TIMEOUT", "LLMK_STATUS_HISTORY_FULL", "LLMK_STATUS_NAN_LOGITS",
                 "LLMK_INVALID_TOKEN"):
        m = re.search(rf"#define {name} \(?(-?(?:0x)?[0-9a-f]+)u?\)?", src)
        assert m, name
        assert int(m.group(1), 0) == getattr(_lib, name), name


def test_host_argument_checks_without_device():
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.llmk_sampler_create(None, 0, 1, 1) == _lib.LLMK_ERR_INVALID_ARGUMENT
    assert lib.llmk_sampler_create(ctypes.byref(h), 0, 0, 1000) == _lib.LLMK_ERR_INVALID_ARGUMENT
    assert "max_batch" in _lib.last_error()
    assert lib.llmk_sampler_create(ctypes.byref(h), 0, 4, (1 << 20) + 1) == _lib.LLMK_ERR_CAPACITY
    assert not h.value
    a = _lib.SampleBatchArgs()
    assert lib.llmk_sample_batch(None, ctypes.byref(a), None) == _lib.LLMK_ERR_INVALID_ARGUMENT
    assert "NULL" in _lib.last_error()
    st = ctypes.c_uint32()
    assert lib.llmk_sampler_status(None, None, ctypes.byref(st)) == _lib.LLMK_ERR_INVALID_ARGUMENT
    assert lib.llmk_history_count_append(None, 1, None, None, None, None, 8, None,
                                         None) == _lib.LLMK_ERR_INVALID_ARGUMENT
    lib.llmk_sampler_destroy(None)  # no-op


def test_product_package_has_no_oracle_path():
    pkg = os.path.join(ROOT, "llm-rs_amd")
    for dp, _, fs in os.walk(pkg):
        for f in fs:
            if f.endswith((".py", ".hip", ".h", ".cpp", "Makefile")):
                txt = open(os.path.join(dp, f)).read()
                assert "llmk_oracle" not in txt and "import oracle" not in txt, f


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libllmk_sampler.so")
    with pytest.raises(OSError, match="no CPU fallback"):
        _lib.load()


def test_sample_params_defaults_follow_types_rs():
    """llm-core/src/types.rs:186-195."""
    p = llmk.SampleParams()
    assert (p.temperature, p.top_p, p.top_k, p.repetition_penalty, p.max_new_tokens) == (1.0, 1.0, 0, 1.0, 512)
    assert (p.presence_penalty, p.frequency_penalty, p.min_p) == (0.0, 0.0, 0.0)


def test_single_row_strides_are_read_as_packed():
    """torch gives a size-1 dimension any stride (np.atleast_2d of a 1-D
    array has stride 0 across rows): one row is read as packed, and a
    one-column tensor needs no unit column stride."""
    import numpy as np
    import torch
    from llmk import sampler as S
    one = torch.from_numpy(np.atleast_2d(np.zeros(3, np.float32)))
    assert one.stride(0) == 0
    assert S._rows(one) and S._row_stride(one) == 3
    assert S._row_stride(torch.zeros(4, 10)) == 10
    assert S._row_stride(torch.zeros(8, 20)[:, 5:15]) == 20
    col = torch.zeros(3, 5)[:, 2:3]
    assert S._rows(col)
    assert not S._rows(torch.zeros(5, 3).t())
