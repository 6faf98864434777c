"""The C-ABI boundary on the CPU: the library loads, exports every symbol include/dotcompute_hip.h
declares, reports errors as documented, and behaves without a device (no compute calls here).
Also checks the product's host generators against the oracle's, since GPU tests and the bench
feed both sides from them."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import oracle
from dotcompute_amd import hip


def test_library_loads_and_reports_abi_version():
    L = hip.load()
    assert L.dc_hip_abi_version() == 1


def test_every_header_symbol_is_exported():
    syms = hip.header_symbols()
    assert len(syms) >= 40
    L = hip.load()
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", hip.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(syms) <= exported
    # every header function has a ctypes signature in the binding
    assert set(syms) <= set(hip.SIGNATURES)


def test_error_strings():
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8):
        assert hip.error_string(code)
    assert "overflow" in hip.error_string(hip.DC_ERR_OVERFLOW)
    assert hip.error_string(-99) == "unknown DotCompute HIP status"


def test_null_and_negative_arguments_are_rejected_before_any_device_work():
    L = hip.load()
    assert L.dc_hip_device_count(None) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_vector_add_f32(None, None, None, None, -1) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_reduce_sum_f32(None, None, 10, None) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_gemm_f32(None, None, None, None, -1, 2, 2) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_spmv_csr_f32(None, None, None, None, None, None, -1, 1, 0) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_gemm_bf16(None, None, None, None, 2, -1, 2) == hip.DC_ERR_INVALID_ARGUMENT
    chain = hip.where_gt0_select_2x_plus_1()
    assert L.dc_hip_linq_where_select_minmax_f32(None, C.byref(chain), None, -1, hip.LINQ_MIN, None,
                                                  None) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_linq_where_select_minmax_f32(None, C.byref(chain), None, 0, 7, None,
                                                  None) == hip.DC_ERR_INVALID_ARGUMENT  # op is neither Min nor Max
    assert L.dc_hip_ctx_create(0, None) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_synchronize(None) == hip.DC_ERR_INVALID_ARGUMENT


def test_no_device_behaviour():
    n = hip.device_count()
    if n > 0:
        pytest.skip("a device is present; covered by the GPU tests")
    ctx = C.c_void_p()
    assert hip.load().dc_hip_ctx_create(0, C.byref(ctx)) == hip.DC_ERR_NO_DEVICE
    with pytest.raises(hip.HipError):
        hip.Context(0)


def test_chain_validation():
    L = hip.load()
    good = hip.where_gt0_select_2x_plus_1()
    assert L.dc_linq_chain_validate(C.byref(good)) == 0
    bad_op = hip.LinqChain.assemble([(40, hip.SRC_IMM, 0)])
    assert L.dc_linq_chain_validate(C.byref(bad_op)) == hip.DC_ERR_UNSUPPORTED
    bad_src = hip.LinqChain.assemble([(hip.LOAD, 9, 0)])
    assert L.dc_linq_chain_validate(C.byref(bad_src)) == hip.DC_ERR_UNSUPPORTED
    pow_prog = hip.LinqChain.assemble([(hip.LOAD, hip.SRC_ELEM, 0), (hip.POW, hip.SRC_IMM, 2.0),
                                       (hip.RPOW, hip.SRC_S0, 0), (hip.MAP, hip.SRC_IMM, 0)])
    assert L.dc_linq_chain_validate(C.byref(pow_prog)) == 0  # MathF.Pow: float32 programs only
    ipow = hip.LinqChain.assemble([(hip.LOAD, hip.SRC_ELEM, 0), (hip.POW, hip.SRC_IMM, 2), (hip.MAP, hip.SRC_IMM, 0)],
                                  int32=True)
    assert L.dc_linq_chain_validate_i32(C.byref(ipow)) == hip.DC_ERR_UNSUPPORTED
    assert L.dc_linq_chain_validate(C.byref(hip.LinqChain.assemble([(hip.RPOW + 1, hip.SRC_IMM, 0)]))) == \
        hip.DC_ERR_UNSUPPORTED
    too_long = hip.LinqChain()
    too_long.n_instr = hip.DC_LINQ_MAX_INSTR + 1
    assert L.dc_linq_chain_validate(C.byref(too_long)) == hip.DC_ERR_INVALID_ARGUMENT
    assert C.sizeof(hip.LinqChain) == 8 + 8 * hip.DC_LINQ_MAX_INSTR  # matches the C struct


def test_product_generators_match_oracle():
    for seed, stream in ((42, 0), (44, 0), (7, 5)):
        assert np.array_equal(hip.gen_uniform_f32(50_000, seed, stream).view(np.uint32),
                              oracle.gen_uniform_f32(50_000, seed, stream).view(np.uint32))
    assert np.array_equal(hip.gen_uniform_f32(1000, 3, 5, True), oracle.gen_uniform_f32(1000, 3, 5, True))
    assert np.array_equal(hip.gen_uniform_i32(50_000, 43, 1), oracle.gen_uniform_i32(50_000, 43, 1))


def test_product_zipf_graph_matches_oracle():
    rp, col, val = hip.gen_zipf_csr(200_000, 42)
    orp, ocol, oval = oracle.gen_zipf_csr(200_000, 42)
    assert np.array_equal(rp, orp) and np.array_equal(col, ocol) and np.array_equal(val, oval)


def test_code_object_ships_next_to_the_library():
    assert os.path.exists(os.path.join(hip.LIB_DIR, "dc_kernels_gfx950.hsaco"))
    assert hip.load().dc_hip_default_module_path().decode().endswith("dc_kernels_gfx950.hsaco")


# The C# struct layouts a managed binding declares ([StructLayout(LayoutKind.Sequential)], natural alignment):
# field -> (offset, size). The C header must place every field exactly there.
CSHARP_LAYOUTS = {
    "dc_hip_device_info": (376, [
        ("name", 0, 256), ("gcn_arch_name", 256, 64), ("device_id", 320, 4), ("compute_units", 324, 4),
        ("wave_size", 328, 4), ("max_threads_per_block", 332, 4), ("clock_khz", 336, 4),
        ("memory_clock_khz", 340, 4), ("memory_bus_width_bits", 344, 4), ("l2_cache_bytes", 348, 4),
        ("total_global_mem", 352, 8), ("lds_per_block", 360, 8), ("pci_bus_id", 368, 4), ("is_gfx950", 372, 4)]),
    "dc_linq_instr": (8, [("op", 0, 1), ("src", 1, 1), ("mode", 2, 1), ("pad", 3, 1), ("imm", 4, 4),
                          ("imm_i32", 4, 4)]),
    "dc_linq_chain": (8 + 8 * 48, [("n_instr", 0, 4), ("flags", 4, 4), ("code", 8, 8 * 48)]),
    "dc_gen_launch": (152, [("work", 0, 8), ("epoch", 8, 4), ("reserved", 12, 4), ("error", 16, 8),
                            ("len", 24, 8 * 16)]),
}


def test_struct_layouts_match_the_csharp_binding(tmp_path):
    """Compiles a probe against include/dotcompute_hip.h and checks offsetof/sizeof of every field
    of the structs the C# binding declares (DeviceInfo, LinqInstr, LinqChain, GenLaunch) against their
    sequential layouts; the ctypes mirrors in dotcompute_amd/hip.py must agree too."""
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "dotcompute_hip.h"', "int main(void) {"]
    for struct, (size, fields) in CSHARP_LAYOUTS.items():
        lines.append(f'printf("{struct} %zu\\n", sizeof({struct}));')
        for f, _, _ in fields:
            lines.append(f'printf("{struct}.{f} %zu %zu\\n", offsetof({struct}, {f}), sizeof((({struct}*)0)->{f}));')
    lines.append("return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(root, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(l.split(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True)
               .stdout.splitlines())
    mirrors = {"dc_hip_device_info": hip.DeviceInfo, "dc_linq_instr": hip.LinqInstr, "dc_linq_chain": hip.LinqChain,
               "dc_gen_launch": hip.GenLaunch}
    for struct, (size, fields) in CSHARP_LAYOUTS.items():
        assert int(got[struct]) == size == C.sizeof(mirrors[struct]), struct
        for f, off, fsize in fields:
            assert got[f"{struct}.{f}"] == f"{off} {fsize}", (struct, f)
            assert getattr(mirrors[struct], f).offset == off, (struct, f)
