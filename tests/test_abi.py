"""The drop-in boundary, checked without a GPU: struct layouts identical to
the reference header, every declared symbol exported, query/capabilities
answering the v1 contract (c/qwanto_decode.c:349-413)."""
import ctypes
import json
import os
import re

import pytest

from abi_layout_probe import probe
from qwanto_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FIXTURE = os.path.join(ROOT, "tests", "golden", "abi_layout.json")


def declared_symbols():
    names = []
    for h in ("qwn_cuda_abi.h", "qwn_hip_ext.h", "qwn_hip_decoder.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        names += re.findall(r"QWN_CUDA_ABI_API\s+[\w\s\*]+?\b(qwn_\w+)\s*\(", text)
    return names


def test_header_layout_matches_reference():
    ref = json.load(open(FIXTURE))
    ours = probe(os.path.join(ROOT, "include", "qwn_cuda_abi.h"))
    assert ours["structs"] == ref["structs"]
    assert ours["constants"] == ref["constants"]


def test_ctypes_mirror_matches_reference():
    ref = json.load(open(FIXTURE))["structs"]
    for name, cls in abi.STRUCTS.items():
        assert ctypes.sizeof(cls) == ref[name]["size"], name
        for field, off in ref[name].items():
            if field != "size":
                assert getattr(cls, field).offset == off, (name, field)


def test_all_declared_symbols_exported(hip_lib):
    names = declared_symbols()
    assert len([n for n in names if n.startswith("qwn_cuda_abi_")]) == 17
    for n in names:
        assert hasattr(hip_lib.lib, n), n
    assert set(abi.EXPORTS) | set(abi.EXT_EXPORTS) | set(abi.DECODER_EXPORTS) == set(names)


def test_extension_struct_layouts():
    """The ctypes mirrors of the extension structs against the C headers,
    compiled here with gcc."""
    import subprocess
    import tempfile
    fields = {"QwnHipGemvGroupRequest": abi.GemvGroupRequest, "QwnHipDecoderDesc": abi.DecoderDesc,
              "QwnHipDecoderStats": abi.DecoderStats, "QwnHipTensorInfo": abi.TensorInfo}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "qwn_hip_ext.h"',
             '#include "qwn_hip_decoder.h"', 'int main(void) {']
    for cname, cls in fields.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as tmp:
        src, exe = os.path.join(tmp, "p.c"), os.path.join(tmp, "p")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-I" + os.path.join(ROOT, "include"), src, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    for line in out.splitlines():
        cname, field, value = line.split()
        cls = fields[cname]
        got = ctypes.sizeof(cls) if field == "size" else getattr(cls, field).offset
        assert got == int(value), (cname, field)


def test_loader_file_name_present():
    # qwnrun dlopen()s "<exe dir>/qwn_cuda.so" (c/qwanto_decode.c:289-301)
    assert os.path.exists(os.path.join(ROOT, "qwanto_amd", "lib", "qwn_cuda.so"))


def test_query_contract(hip_lib):
    info = hip_lib.query()
    assert info.header.abi_version == 1
    assert info.header.struct_size >= ctypes.sizeof(abi.AbiInfo)
    assert info.hypervsq2_block_bytes == 74 and info.hypervsq2_block_elements == 256
    need = (abi.CAP_HYPERVSQ2_GEMV | abi.CAP_HYPERVSQ2_GEMM | abi.CAP_Q8_KV | abi.CAP_Q4_0_GEMV |
            abi.CAP_F16_GEMV | abi.CAP_BF16_GEMV | abi.CAP_DEVICE_POINTERS)
    assert info.capability_bits & need == need
    assert info.abi_name == b"qwn_cuda_hypervsq2"
    assert info.max_resident_tensors == 512


def test_query_rejects_bad_header(hip_lib):
    info = abi.AbiInfo()
    info.header.abi_version = 2
    assert hip_lib.lib.qwn_cuda_abi_query(ctypes.byref(info)) == -1
    assert "invalid" in hip_lib.last_error()
    small = abi.AbiInfo()
    small.header.struct_size = 8
    assert hip_lib.lib.qwn_cuda_abi_query(ctypes.byref(small)) == -1


def test_null_arguments_rejected(hip_lib):
    lib = hip_lib.lib
    assert lib.qwn_cuda_abi_context_create(None, None) == -1
    assert lib.qwn_cuda_abi_upload_tensor(None, None, None) == -1
    assert lib.qwn_cuda_abi_hypervsq2_gemv(None, None, None) == -1
    assert lib.qwn_cuda_abi_last_error(None, 0) == -1


def test_no_cpu_fallback_in_package():
    """The product path must fail loudly without the HIP library."""
    with pytest.raises(FileNotFoundError):
        abi.Library("/nonexistent/libqwn_hip.so")
    for dirpath, _, files in os.walk(os.path.join(ROOT, "qwanto_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".c", ".cpp")):
                text = open(os.path.join(dirpath, f), errors="replace").read()
                assert "import oracle" not in text and "from oracle" not in text, f
