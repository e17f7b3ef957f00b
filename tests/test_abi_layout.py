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


def test_extension_ctypes_mirror_matches_header(tmp_path):
    """The extension header's structures (no reference counterpart) as gcc lays
    them out, against the ctypes mirror the tests call through."""
    structs = {"xvram_amd_epilogue_v1": abi.EpilogueV1, "xvram_amd_device_info_v1": abi.DeviceInfoV1,
               "xvram_amd_sgemm_v1": abi.SgemmDeviceV1, "xvram_amd_ext_v1": abi.ExtV1}
    lines = ["#include <xvram/xvram_amd_ext.h>", "#include <stdio.h>", "#include <stddef.h>",
             "int main(void){"]
    for name, cls in structs.items():
        lines.append(f'printf("S {name} %zu\\n", sizeof({name}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("O {name} {field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0;}")
    src = tmp_path / "ext.c"
    src.write_text("\n".join(lines))
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{ROOT}/include", str(src), "-o",
                    str(tmp_path / "ext")], check=True)
    out = subprocess.run([str(tmp_path / "ext")], check=True, capture_output=True, text=True).stdout
    for line in out.splitlines():
        parts = line.split()
        cls = structs[parts[1]]
        if parts[0] == "S":
            assert ctypes.sizeof(cls) == int(parts[2]), parts[1]
        else:
            assert getattr(cls, parts[2]).offset == int(parts[3]), (parts[1], parts[2])


def test_device_gemm_rules_without_a_gpu():
    """sgemm_device's (and sgemm_device_no_alloc's) descriptor checks
    (INVALID_ARGUMENT / INCOMPATIBLE_ABI) run before any device work; a valid
    descriptor is UNSUPPORTED in the host simulation, which has no device
    memory."""
    lib = xv.Library(xv.HOSTSIM_LIB)
    for call in (lib.ext.sgemm_device, lib.ext.sgemm_device_no_alloc):
        check_device_gemm_rules(call)


def check_device_gemm_rules(call):
    def valid():
        d = abi.sgemm_device_init()
        d.a, d.b, d.c = 4096, 8192, 12288  # 16-byte aligned stand-ins, never dereferenced
        d.m, d.n, d.k = 256, 256, 256
        d.lda = d.ldb = d.ldc = 256
        return d

    assert call(ctypes.byref(valid()), None) == abi.UNSUPPORTED
    assert call(None, None) == abi.INCOMPATIBLE_ABI
    d = valid()
    d.struct_size = 8
    assert call(ctypes.byref(d), None) == abi.INCOMPATIBLE_ABI
    bad = [("flags", 1), ("operation_a", 2), ("bias_axis", 3), ("activation", 2), ("a", None),
           ("m", 0), ("k", 1 << 31), ("lda", 128), ("ldc", 258), ("b", 8200),
           ("bias_axis", abi.BIAS_PER_ROW), ("workspace_bytes", 64)]
    for field, value in bad:
        d = valid()
        setattr(d, field, value)
        assert call(ctypes.byref(d), None) == abi.INVALID_ARGUMENT, field
    d = valid()
    d.operation_a = abi.OP_T  # A stored k x m: lda must cover k, B (op N) k x n: ldb too
    d.k, d.lda, d.ldb = 512, 256, 512
    assert call(ctypes.byref(d), None) == abi.INVALID_ARGUMENT
    d.lda = 512
    assert call(ctypes.byref(d), None) == abi.UNSUPPORTED


def _elf_exports(path):
    """Defined dynamic symbols as the reference's export contract reads them
    (tests/contract/sdk_export_contract.py:66-99): `nm -D --defined-only
    --format=posix`; an absolute symbol named like a version node is that
    node, every other line is an export, `sym@@NODE` carries its version."""
    out = subprocess.run(["nm", "-D", "--defined-only", "--format=posix", path], check=True,
                         capture_output=True, text=True).stdout
    exports, nodes, versions = set(), set(), {}
    for line in out.splitlines():
        fields = line.split()
        if len(fields) < 2:
            continue
        raw, kind = fields[0], fields[1].upper()
        if kind == "A" and "@" not in raw:
            nodes.add(raw)
            continue
        symbol, sep, version = raw.partition("@")
        exports.add(symbol)
        if sep:
            versions[symbol] = version.lstrip("@")
    return exports, nodes, versions


def _version_definitions(path):
    """Non-base ELF version definitions (.gnu.version_d). Newer GNU ld no
    longer emits the absolute version-node symbol that older nm output lists,
    so the node's presence is read from the section itself."""
    out = subprocess.run(["readelf", "-V", "-W", path], check=True, capture_output=True,
                         text=True).stdout
    nodes = set()
    in_defs = False
    for line in out.splitlines():
        if line.startswith("Version definition section"):
            in_defs = True
            continue
        if in_defs and line.startswith("Version "):
            break
        if in_defs and "Name:" in line and "Flags: BASE" not in line:
            nodes.add(line.split("Name:")[1].split()[0])
    return nodes


def test_product_exports_exactly_the_reference_symbol():
    """The reference's contract (sdk_export_contract.py:13-14,106-125): the
    export set is exactly {xvram_get_api}, at ELF version XVRAM_0.1, and the
    XVRAM_0.1 node exists. The extension table adds no symbol."""
    exports, nodes, versions = _elf_exports(xv.PRODUCT_LIB)
    assert exports == {"xvram_get_api"}
    assert nodes <= {"XVRAM_0.1"}
    assert _version_definitions(xv.PRODUCT_LIB) == {"XVRAM_0.1"}
    assert versions == {"xvram_get_api": "XVRAM_0.1"}


def test_hostsim_exports_the_same_entry_point():
    exports, nodes, versions = _elf_exports(xv.HOSTSIM_LIB)
    assert versions["xvram_get_api"] == "XVRAM_0.1"
    # Only the simulation's own test hooks besides the entry point.
    assert all(s == "xvram_get_api" or s.startswith("xvram_hostsim_") for s in exports)


@pytest.mark.parametrize("path", [xv.PRODUCT_LIB, xv.HOSTSIM_LIB])
def test_extension_table_through_get_api(path):
    """The extension table is one more version of xvram_get_api, with the
    v1 table's argument rules; other unknown versions stay incompatible."""
    lib = xv.Library(path)
    ext = abi.ExtV1()
    size = ctypes.sizeof(ext)
    assert lib.get_api(abi.EXT_ABI_VERSION_1, size, ctypes.byref(ext)) == abi.SUCCESS
    assert ext.struct_size == size and ext.ext_version == abi.EXT_VERSION_2
    assert ctypes.cast(ext.gemm_plan_create_epilogue, ctypes.c_void_p).value
    assert ctypes.cast(ext.device_get_info, ctypes.c_void_p).value
    assert ctypes.cast(ext.sgemm_device, ctypes.c_void_p).value
    assert ctypes.cast(ext.sgemm_device_no_alloc, ctypes.c_void_p).value
    assert list(ext.reserved) == [0]
    assert lib.get_api(abi.EXT_ABI_VERSION_1, size - 1, ctypes.byref(ext)) == abi.INVALID_ARGUMENT
    assert lib.get_api(abi.EXT_ABI_VERSION_1, size, None) == abi.INVALID_ARGUMENT
    for version in (abi.EXT_ABI_VERSION_1 + 1, abi.EXT_ABI_VERSION_1 - 1, 0x58410000, 1 << 31):
        assert lib.get_api(version, 4096, (ctypes.c_uint8 * 4096)()) == abi.INCOMPATIBLE_ABI


def test_export_parser_rejects_extra_symbols():
    """The parser above must see what the reference contract rejects."""
    import types
    fake = ("XVRAM_0.1 A 0\nXVRAM_AMD_EXT_1 A 0\nxvram_get_api@@XVRAM_0.1 T 100\n"
            "xvram_amd_get_ext@@XVRAM_AMD_EXT_1 T 200\n")
    real_run = subprocess.run
    try:
        subprocess.run = lambda *a, **k: types.SimpleNamespace(stdout=fake)
        exports, nodes, versions = _elf_exports("unused")
    finally:
        subprocess.run = real_run
    assert exports == {"xvram_get_api", "xvram_amd_get_ext"}
    assert nodes == {"XVRAM_0.1", "XVRAM_AMD_EXT_1"}
    assert versions["xvram_amd_get_ext"] == "XVRAM_AMD_EXT_1"


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
