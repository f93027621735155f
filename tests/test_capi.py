"""The C-ABI libraries on the CPU: every symbol the headers declare is exported, host-only entry points work
without a GPU, errors come back as status codes, and the product libraries do not link the oracle."""
import ctypes
import os
import re
import subprocess

import pytest

import veckern_amd as vk
from veckern_amd import host

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "veckern_amd", "lib")


def declared(header, prefix):
    text = open(os.path.join(ROOT, "include", "veckern", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(rf"\b({prefix}\w+)\s*\(", text)))


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_libveckern_exports_every_declared_entry_point():
    names = declared("veckern.h", "vk_")
    assert len(names) >= 18
    syms = exported(os.path.join(LIB, "libveckern.so"))
    missing = [n for n in names if n not in syms]
    assert not missing, missing
    # nothing else is exported: internal kernels and helpers stay hidden behind the C ABI
    extra = sorted(s for s in syms if s.startswith("vk_") and s not in names)
    assert not extra, extra


def test_host_library_exports_every_declared_entry_point():
    names = declared("host.h", "vkh_")
    syms = exported(os.path.join(LIB, "libveckern_cpu.so"))
    assert not [n for n in names if n not in syms]


def test_cpp_api_library_exports_the_searcher():
    out = subprocess.run(["nm", "-DC", "--defined-only", os.path.join(LIB, "libveckern_gpu.so")],
                         capture_output=True, text=True, check=True).stdout
    for sym in ("veckern::gpu::PQSearcher::PQSearcher", "veckern::gpu::PQSearcher::search",
                "veckern::gpu::PQSearcher::distances", "veckern::gpu::PQSearcher::set_tuning",
                "veckern::gpu::PQSearcher::last_launch", "veckern::gpu::device_info", "veckern::gpu::variant_name",
                "veckern::gpu::is_fused", "veckern::gpu::Reranker::Reranker", "veckern::gpu::Reranker::rerank",
                "veckern::gpu::IVFSearcher::IVFSearcher", "veckern::gpu::IVFSearcher::search",
                "veckern::gpu::assign_lists", "veckern::gpu::encode", "veckern::gpu::train"):
        assert sym in out, sym


def test_product_libraries_do_not_link_the_oracle():
    for name in os.listdir(LIB):
        path = os.path.join(LIB, name)
        deps = subprocess.run(["ldd", path], capture_output=True, text=True).stdout
        assert "vk_oracle" not in deps and "vkref" not in deps, name
        und = subprocess.run(["nm", "-D", "--undefined-only", path], capture_output=True, text=True).stdout
        assert "vko_" not in und and "vkref_" not in und, name
    for py in os.listdir(os.path.join(ROOT, "veckern_amd")):
        if py.endswith(".py"):
            src = open(os.path.join(ROOT, "veckern_amd", py)).read()
            assert "oracle" not in re.sub(r'""".*?"""', "", src, flags=re.S).replace("#", "\n#"), py


def test_variant_registry():
    names = [vk.variant_name(v) for v in vk.ScanVariant]
    assert names == ["v0_global_lut", "v1_shared_lut", "v2_shared_lut_vec", "v3_interleaved", "v4_fused",
                     "v5_fused_reg", "v6_fused_vec", "v7_fused_vec_mq", "v8_fused_warp", "v9_fused_warp_f16"]
    assert [vk.is_fused(v) for v in vk.ScanVariant] == [False] * 4 + [True] * 6
    assert [vk.needs_m16(v) for v in vk.ScanVariant] == [False, False, True, False, False, False, True, True, True,
                                                         True]
    assert vk.variant_name(10) == "unknown" and vk.variant_name(-1) == "unknown"


def test_tuning_defaults_and_validation():
    t = vk.library()
    c = vk._Tuning()
    t.vk_tuning_default(ctypes.byref(c))
    assert (c.scan_threads, c.blocks_per_query, c.queries_per_block, c.vectors_per_step) == (256, 0, 2, 4)
    vk.validate_tuning(vk.Tuning())
    for good in (vk.Tuning(32, 0, 1, 1), vk.Tuning(1024, 5, 8, 2), vk.Tuning(96, 0, 4, 4)):
        vk.validate_tuning(good)
    for bad in (vk.Tuning(100, 0, 2, 1), vk.Tuning(256, -1, 2, 1), vk.Tuning(256, 0, 3, 1), vk.Tuning(256, 0, 2, 3),
                vk.Tuning(16, 0, 2, 1), vk.Tuning(2048, 0, 2, 1)):
        with pytest.raises(vk.VkError):
            vk.validate_tuning(bad)


def test_dispatched_k():
    assert [vk.dispatched_k(k) for k in (1, 8, 9, 16, 17, 33, 65, 128)] == [8, 8, 16, 16, 32, 64, 128, 128]
    with pytest.raises(vk.VkInvalidArgument):
        vk.dispatched_k(129)


def test_errors_come_back_as_status_codes_without_a_gpu():
    lib = vk.library()
    h = ctypes.c_void_p()
    import numpy as np
    cent = np.zeros((16, 256, 8), dtype=np.float32)
    codes = np.zeros((10, 16), dtype=np.uint8)
    # invalid shapes are rejected before any device call
    rc = lib.vk_searcher_create(cent.ctypes.data, 130, 16, codes.ctypes.data, 10, ctypes.byref(h))
    assert rc == vk.VK_ERR_RUNTIME and b"multiple of m" in lib.vk_last_error()
    rc = lib.vk_searcher_create(cent.ctypes.data, 128, 16, codes.ctypes.data, 0, ctypes.byref(h))
    assert rc == vk.VK_ERR_RUNTIME and b"int32" in lib.vk_last_error()
    rc = lib.vk_searcher_create(None, 128, 16, codes.ctypes.data, 10, ctypes.byref(h))
    assert rc == vk.VK_ERR_RUNTIME
    assert lib.vk_search(None, None, 0, 10, 8, None, None) == vk.VK_ERR_RUNTIME
    lib.vk_searcher_destroy(None)  # accepted
    assert lib.vk_abi_version() == 1


def test_host_tools_thread_count():
    assert host.max_threads() >= 1
