"""The drop-in boundary: header layout, the single export, the function table
and the ABI entry-point argument rules (no GPU needed: nothing here computes)."""
import ctypes
import os
import subprocess
import textwrap

import pytest

import xvram_amd as xv
from xvram_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Sizes of the reference header's structures on x86-64
# (include/xvram/xvram.h of TheLitis/xVRAM, measured with gcc).
REFERENCE_SIZES = {
    "xvram_error_info_v1": 440, "xvram_session_config_v1": 112,
    "xvram_allocation_desc_v1": 48, "xvram_allocation_info_v1": 56,
    "xvram_access_range_v1": 32, "xvram_prefetch_desc_v1": 48,
    "xvram_resolved_range_v1": 40, "xvram_transaction_context_v1": 80,
    "xvram_transaction_desc_v1": 72, "xvram_operation_info_v1": 96,
    "xvram_matrix_v1": 72, "xvram_gemm_desc_v1": 320, "xvram_gemm_plan_info_v1": 104,
    "xvram_session_telemetry_v1": 320, "xvram_api_v1": 336,
}
REFERENCE_OFFSETS = {
    ("xvram_gemm_desc_v1", "a"): 8, ("xvram_gemm_desc_v1", "b"): 80,
    ("xvram_gemm_desc_v1", "c"): 152, ("xvram_gemm_desc_v1", "operation_a"): 224,
    ("xvram_gemm_desc_v1", "alpha"): 240, ("xvram_gemm_desc_v1", "beta"): 248,
    ("xvram_gemm_desc_v1", "workspace_cap_bytes"): 256,
    ("xvram_gemm_desc_v1", "deadline_ms"): 264, ("xvram_gemm_desc_v1", "tile_m_hint"): 272,
    ("xvram_api_v1", "gemm_plan_create"): 128, ("xvram_api_v1", "gemm_submit"): 144,
    ("xvram_api_v1", "operation_release"): 200, ("xvram_api_v1", "reserved"): 208,
}
CTYPES = {
    "xvram_error_info_v1": abi.ErrorInfo, "xvram_session_config_v1": abi.SessionConfig,
    "xvram_allocation_desc_v1": abi.AllocationDesc, "xvram_allocation_info_v1": abi.AllocationInfo,
    "xvram_access_range_v1": abi.AccessRange, "xvram_prefetch_desc_v1": abi.PrefetchDesc,
    "xvram_resolved_range_v1": abi.ResolvedRange,
    "xvram_transaction_context_v1": abi.TransactionContext,
    "xvram_transaction_desc_v1": abi.TransactionDesc, "xvram_operation_info_v1": abi.OperationInfo,
    "xvram_matrix_v1": abi.Matrix, "xvram_gemm_desc_v1": abi.GemmDesc,
    "xvram_gemm_plan_info_v1": abi.GemmPlanInfo,
    "xvram_session_telemetry_v1": abi.SessionTelemetry, "xvram_api_v1": abi.ApiV1,
}


@pytest.fixture(scope="module")
def header_layout(tmp_path_factory):
    """sizeof/offsetof of every structure as gcc computes them from include/xvram/xvram.h."""
    d = tmp_path_factory.mktemp("layout")
    lines = ["#include <xvram/xvram.h>", "#include <stdio.h>", "#include <stddef.h>", "int main(void){"]
    for name in REFERENCE_SIZES:
        lines.append(f'printf("S {name} %zu\\n", sizeof({name}));')
    for (s, f) in REFERENCE_OFFSETS:
        lines.append(f'printf("O {s} {f} %zu\\n", offsetof({s}, {f}));')
    lines.append("return 0;}")
    src = d / "layout.c"
    src.write_text("\n".join(lines))
    exe = d / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{ROOT}/include", str(src), "-o",
                    str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    sizes, offsets = {}, {}
    for line in out.splitlines():
        parts = line.split()
        if parts[0] == "S":
            sizes[parts[1]] = int(parts[2])
        else:
            offsets[(parts[1], parts[2])] = int(parts[3])
    return sizes, offsets


def test_header_matches_reference_layout(header_layout):
    sizes, offsets = header_layout
    assert sizes == REFERENCE_SIZES
    assert offsets == REFERENCE_OFFSETS


def test_header_compiles_as_cplusplus(tmp_path):
    src = tmp_path / "t.cpp"
    src.write_text("#include <xvram/xvram.h>\nint main(){xvram_gemm_desc_v1 d = XVRAM_GEMM_DESC_V1_INIT;"
                   "xvram_session_config_v1 c = XVRAM_SESSION_CONFIG_V1_INIT; return (int)(d.alpha - 1.0)"
                   " + (int)c.staging_slots - 4;}\n")
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", f"-I{ROOT}/include", str(src), "-o",
                    str(tmp_path / "t")], check=True)
    assert subprocess.run([str(tmp_path / "t")]).returncode == 0


def test_ctypes_mirror_matches_header(header_layout):
    sizes, offsets = header_layout
    for name, cls in CTYPES.items():
        assert ctypes.sizeof(cls) == sizes[name], name
    for (s, f), off in offsets.items():
        assert getattr(CTYPES[s], f).offset == off, (s, f)


@pytest.mark.parametrize("path", [xv.PRODUCT_LIB, xv.HOSTSIM_LIB])
def test_exports(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True,
                         text=True).stdout
    symbols = sorted(line.split()[-1] for line in out.splitlines() if " T " in line)
    if path == xv.PRODUCT_LIB:
        # The reference's one export, versioned like its export map, plus this
        # build's extension table in a version node of its own.
        assert symbols == ["xvram_amd_get_ext@@XVRAM_AMD_EXT_1", "xvram_get_api@@XVRAM_0.1"]
    else:
        assert "xvram_get_api@@XVRAM_0.1" in symbols


def test_product_library_loads_without_gpu():
    lib = xv.Library(xv.PRODUCT_LIB)
    api = lib.api
    assert api.struct_size == ctypes.sizeof(abi.ApiV1)
    assert api.abi_version == 1
    for name, _ in abi.ApiV1._fields_:
        if name not in ("struct_size", "abi_version", "reserved"):
            assert ctypes.cast(getattr(api, name), ctypes.c_void_p).value, name
    assert list(api.reserved) == [0] * 16


def test_get_api_argument_rules():
    lib = xv.Library(xv.PRODUCT_LIB)
    buf = (ctypes.c_uint8 * 512)()
    assert lib.get_api(1, 336, buf) == abi.SUCCESS
    assert lib.get_api(1, 335, buf) == abi.INVALID_ARGUMENT
    assert lib.get_api(1, 336, None) == abi.INVALID_ARGUMENT
    assert lib.get_api(0, 336, buf) == abi.INCOMPATIBLE_ABI
    assert lib.get_api(3, 336, buf) == abi.INCOMPATIBLE_ABI


def test_status_names_match_reference():
    lib = xv.Library(xv.PRODUCT_LIB)
    for code, name in abi.STATUS.items():
        assert lib.status_name(code) == name
    assert lib.status_name(20) == "unknown"
    assert lib.status_name(0xFFFFFFFF) == "unknown"


def test_c_consumer_compiles_and_links(tmp_path):
    """A C caller written against the header links against libxvram.so with no
    HIP headers (the reference's package consumer, tests/package_consumer/main.c)."""
    src = tmp_path / "consumer.c"
    src.write_text(textwrap.dedent("""
        #include <xvram/xvram.h>
        #include <stdio.h>
        int main(void) {
          xvram_api_v1 api;
          if (xvram_get_api(XVRAM_ABI_VERSION_1, sizeof(api), &api) != XVRAM_STATUS_SUCCESS) return 1;
          if (api.struct_size != sizeof(api) || api.abi_version != XVRAM_ABI_VERSION_1) return 2;
          printf("%s\\n", api.status_name(XVRAM_STATUS_BUDGET_PRESSURE));
          return 0;
        }
    """))
    exe = tmp_path / "consumer"
    libdir = os.path.dirname(xv.PRODUCT_LIB)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{ROOT}/include", str(src), "-o",
                    str(exe), f"-L{libdir}", "-lxvram", f"-Wl,-rpath,{libdir}"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert out.strip() == "budget_pressure"
