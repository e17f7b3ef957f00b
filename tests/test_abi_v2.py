"""ABI v2 (include/xvram/xvram_v2.h): header layout against the reference's, the
v2 table and xvram_get_api(2) rules (src/sdk/api.cpp:1002-1035), config
validation order (src/sdk/api.cpp:209-233), and the compression policy of this
build: DISABLED sessions are v1 sessions, ADAPTIVE/CAPACITY are UNSUPPORTED.
Sessions run over the hostsim library; nothing here needs a GPU."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# sizeof / offsetof measured from the reference header (include/xvram/xvram_v2.h) with gcc.
REFERENCE_V2 = {"config": 224, "telemetry": 680, "api": 464, "config.compression_mode": 120,
                "telemetry.logical_bytes": 328, "api.session_create_v2": 336,
                "telemetry.verification_nanoseconds": 608}


def test_v2_header_layout(tmp_path):
    src = tmp_path / "v2.c"
    src.write_text("""
#include <xvram/xvram_v2.h>
#include <stdio.h>
#include <stddef.h>
int main(void) {
  xvram_session_config_v2 c = XVRAM_SESSION_CONFIG_V2_INIT;
  printf("%zu %zu %zu %zu %zu %zu %zu %u\\n", sizeof(xvram_session_config_v2),
         sizeof(xvram_session_telemetry_v2), sizeof(xvram_api_v2),
         offsetof(xvram_session_config_v2, compression_mode),
         offsetof(xvram_session_telemetry_v2, logical_bytes),
         offsetof(xvram_api_v2, session_create_v2),
         offsetof(xvram_session_telemetry_v2, verification_nanoseconds), c.compression_mode);
  return 0;
}
""")
    exe = tmp_path / "v2"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{ROOT}/include", str(src), "-o",
                    str(exe)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True,
                                           text=True).stdout.split()]
    assert vals[:7] == [REFERENCE_V2[k] for k in (
        "config", "telemetry", "api", "config.compression_mode", "telemetry.logical_bytes",
        "api.session_create_v2", "telemetry.verification_nanoseconds")]
    assert vals[7] == abi.COMPRESSION_ADAPTIVE
    assert ctypes.sizeof(abi.SessionConfigV2) == 224
    assert ctypes.sizeof(abi.SessionTelemetryV2) == 680
    assert ctypes.sizeof(abi.ApiV2) == 464


def v2_table(path):
    lib = xv.Library(path)
    api = abi.ApiV2()
    assert lib.get_api(2, ctypes.sizeof(api), ctypes.byref(api)) == abi.SUCCESS
    return lib, api


@pytest.fixture(params=[xv.PRODUCT_LIB, xv.HOSTSIM_LIB], ids=["product", "hostsim"])
def v2(request):
    return v2_table(request.param)


@pytest.fixture()
def v2_sim():
    """Sessions need a device: the hostsim library provides one on the CPU."""
    return v2_table(xv.HOSTSIM_LIB)


def test_v2_table(v2):
    lib, api = v2
    assert api.v1.struct_size == ctypes.sizeof(abi.ApiV2)
    assert api.v1.abi_version == 2
    assert list(api.reserved) == [0] * 14
    for name, _ in abi.ApiV1._fields_:
        if name not in ("struct_size", "abi_version", "reserved"):
            mine = ctypes.cast(getattr(api.v1, name), ctypes.c_void_p).value
            assert mine == ctypes.cast(getattr(lib.api, name), ctypes.c_void_p).value, name
    buf = (ctypes.c_uint8 * 512)()
    assert lib.get_api(2, 463, buf) == abi.INVALID_ARGUMENT
    assert lib.get_api(2, 464, None) == abi.INVALID_ARGUMENT


def create_v2(api, cfg):
    handle = ctypes.c_void_p()
    status = api.session_create_v2(ctypes.byref(cfg), ctypes.byref(handle))
    return status, handle


def test_v2_config_validation_and_modes(v2_sim):
    lib, api = v2_sim
    lib.dll.xvram_hostsim_reset()
    cfg = abi.session_config_v2_init()
    assert create_v2(api, cfg)[0] == abi.UNSUPPORTED          # the INIT default is ADAPTIVE
    cfg.compression_mode = abi.COMPRESSION_CAPACITY
    assert create_v2(api, cfg)[0] == abi.UNSUPPORTED
    for field, value, status in [("compression_mode", 3, abi.INVALID_ARGUMENT),
                                 ("compression_codec", 2, abi.INVALID_ARGUMENT),
                                 ("compression_workspace_cap_bytes", 0, abi.INVALID_ARGUMENT),
                                 ("codec_slots", 1, abi.INVALID_ARGUMENT),
                                 ("codec_slots", 9, abi.INVALID_ARGUMENT),
                                 ("codec_workers", 0, abi.INVALID_ARGUMENT),
                                 ("codec_workers", 9, abi.INVALID_ARGUMENT),
                                 ("flags", 1, abi.INVALID_ARGUMENT),
                                 ("struct_size", 223, abi.INCOMPATIBLE_ABI)]:
        c = abi.session_config_v2_init()
        c.compression_mode = abi.COMPRESSION_DISABLED
        setattr(c, field, value)
        assert create_v2(api, c)[0] == status, field
    c = abi.session_config_v2_init()
    c.compression_mode = abi.COMPRESSION_DISABLED
    c.reserved[7] = 1
    assert create_v2(api, c)[0] == abi.INVALID_ARGUMENT
    c.reserved[7] = 0
    c.v1.staging_slots = 1  # the embedded v1 config is validated too
    assert create_v2(api, c)[0] == abi.INVALID_ARGUMENT


def test_v2_disabled_session_and_telemetry(v2_sim):
    lib, api = v2_sim
    lib.dll.xvram_hostsim_reset()
    cfg = abi.session_config_v2_init()
    cfg.compression_mode = abi.COMPRESSION_DISABLED
    cfg.v1.chunk_size_bytes = 16 << 10
    cfg.v1.cache_target_bytes = 8 * (16 << 10)
    cfg.v1.device_headroom_bytes = 0
    cfg.v1.workspace_cap_bytes = 0
    status, handle = create_v2(api, cfg)
    assert status == abi.SUCCESS
    s = xv.Session.__new__(xv.Session)  # wrap the handle for the v1 helpers
    s.lib, s.api, s.handle, s.config = lib, lib.api, handle, cfg.v1
    try:
        a = s.allocation(3000)
        b = s.allocation(5000)
        a.write(np.arange(3000, dtype=np.uint8))
        s.execute_transaction([xv.access(a, 0, 3000, abi.ACCESS_READ_WRITE)], lambda v: None)
        a.read()  # the written chunk stays cached, dirty, until read back
        b.release()
        t2 = abi.SessionTelemetryV2()
        t2.struct_size = ctypes.sizeof(t2)
        assert api.session_get_telemetry_v2(handle, ctypes.byref(t2)) == abi.SUCCESS
        t1 = s.telemetry()
        assert t2.struct_size == ctypes.sizeof(t2)
        assert t2.v1.bytes_h2d == t1.bytes_h2d > 0 and t2.v1.bytes_d2h == t1.bytes_d2h > 0
        assert t2.logical_bytes == t2.host_stored_bytes == t2.host_raw_bytes == 3000
        assert t2.host_stored_peak_bytes == 8000
        assert t2.logical_h2d_bytes == t2.pcie_h2d_bytes == t1.bytes_h2d
        assert t2.logical_d2h_bytes == t2.pcie_d2h_bytes == t1.bytes_d2h
        assert t2.compression_attempts == t2.host_compressed_bytes == 0
        small = abi.SessionTelemetryV2()
        small.struct_size = 100
        assert api.session_get_telemetry_v2(handle, ctypes.byref(small)) == abi.INVALID_ARGUMENT
    finally:
        s.close()
        s.release()
