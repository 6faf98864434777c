"""ctypes binding of ``libdotcompute_hip.so`` (the C ABI in ``include/dotcompute_hip.h``).

This is the same boundary the managed HIP backend binds with ``[LibraryImport]``; tests and
``bench.py`` drive the kernels through it. Nothing here falls back to the CPU: if the library is
missing, or no gfx950 device is present, the calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libdotcompute_hip.so")
BENCH_LIB_PATH = os.path.join(LIB_DIR, "libdotcompute_bench.so")  # measurement-only probes
PROBE_COPY, PROBE_READ2_WRITE1, PROBE_READ = 0, 1, 2  # dc_bench_stream_probe kinds
HEADER = os.path.join(os.path.dirname(PKG), "include", "dotcompute_hip.h")

DC_OK = 0
DC_ERR_INVALID_ARGUMENT = -1
DC_ERR_NO_DEVICE = -2
DC_ERR_UNSUPPORTED = -3
DC_ERR_OVERFLOW = -4
DC_ERR_MISALIGNED = -5
DC_ERR_DIMENSION = -6
DC_ERR_OUT_OF_MEMORY = -7
DC_ERR_NOT_FOUND = -8
DC_ERR_COMPILE = -9

# dc_linq_strategy: which kernel dc_hip_linq_where_select_f32 runs for an input
STRATEGY_LOOKBACK = 0
STRATEGY_ROUNDS = 1
LINQ_FLAG_ORDERED_GRID = 1  # dc_linq_chain.flags: run ToArray on the ticket-ordered lookback grid
LINQ_FLAG_INTERPRET = 2     # dc_linq_chain.flags: never compile the program at run time
LINQ_COMPILE_MIN_ELEMENTS = 1 << 22  # ToArray inputs from this size run interpreted programs compiled
LINQ_ELEMENT_F32, LINQ_ELEMENT_I32 = 0, 1

# dc_linq_minmax: which terminal dc_hip_linq_where_select_minmax_f32 computes
LINQ_MIN = 0
LINQ_MAX = 1
# Aggregate((acc, x) => MathF.Min(acc, x)) / MathF.Max: IEEE minimum / maximum folds
LINQ_FOLD_MIN = 2
LINQ_FOLD_MAX = 3

DC_LINQ_MAX_INSTR = 48

# dc_linq_op
NOP, LOAD, ADD, SUB, RSUB, MUL, DIV, RDIV, MIN, MAX, NEG, ABS, SQRT, STORE_S0, STORE_S1 = range(15)
REM, RREM, FLOOR, CEIL, ROUND = range(15, 20)
CMP_GT, CMP_GE, CMP_LT, CMP_LE, CMP_EQ, CMP_NE, PNOT, PSTORE, PAND_Q, POR_Q, FILTER, MAP = range(20, 32)
POW, RPOW = range(32, 34)
# dc_linq_src
SRC_IMM, SRC_ELEM, SRC_S0, SRC_S1 = range(4)
# dc_linq_cmp_mode
CMP_SET, CMP_AND, CMP_OR = range(3)
# int32 chains: fault word = -1 or 4 * index + kind
LINQ_FAULT_NONE, LINQ_FAULT_DIVIDE_BY_ZERO, LINQ_FAULT_OVERFLOW = -1, 1, 2


class DeviceInfo(C.Structure):
    _fields_ = [
        ("name", C.c_char * 256),
        ("gcn_arch_name", C.c_char * 64),
        ("device_id", C.c_int32),
        ("compute_units", C.c_int32),
        ("wave_size", C.c_int32),
        ("max_threads_per_block", C.c_int32),
        ("clock_khz", C.c_int32),
        ("memory_clock_khz", C.c_int32),
        ("memory_bus_width_bits", C.c_int32),
        ("l2_cache_bytes", C.c_int32),
        ("total_global_mem", C.c_int64),
        ("lds_per_block", C.c_int64),
        ("pci_bus_id", C.c_int32),
        ("is_gfx950", C.c_int32),
    ]


DC_GEN_MAX_BUFFERS = 16
DC_GEN_BLOCK = 256
DC_GEN_ERR_INDEX, DC_GEN_ERR_DIVIDE_BY_ZERO, DC_GEN_ERR_OVERFLOW = 0, 1, 2


class GenLaunch(C.Structure):
    """dc_gen_launch: the launch block a generated [Kernel] takes after its buffers and scalars."""
    _fields_ = [("work", C.c_int64), ("epoch", C.c_uint32), ("reserved", C.c_uint32),
                ("error", C.c_void_p), ("len", C.c_int64 * DC_GEN_MAX_BUFFERS)]


class _LinqImm(C.Union):
    _fields_ = [("imm", C.c_float), ("imm_i32", C.c_int32)]


class LinqInstr(C.Structure):
    _anonymous_ = ("u",)
    _fields_ = [("op", C.c_uint8), ("src", C.c_uint8), ("mode", C.c_uint8), ("pad", C.c_uint8), ("u", _LinqImm)]


class LinqChain(C.Structure):
    _fields_ = [("n_instr", C.c_int32), ("flags", C.c_int32), ("code", LinqInstr * DC_LINQ_MAX_INSTR)]

    @classmethod
    def assemble(cls, instrs, int32: bool = False) -> "LinqChain":
        """Build a program from (op, src, imm[, mode]) tuples; int32=True stores the constants as
        int32 (a program for the _i32 entry points)."""
        ch = cls()
        if len(instrs) > DC_LINQ_MAX_INSTR:
            raise ValueError("program too long")
        ch.n_instr = len(instrs)
        ch.flags = 0
        for i, t in enumerate(instrs):
            op, src, imm = t[0], t[1], t[2]
            mode = t[3] if len(t) > 3 else CMP_SET
            ins = LinqInstr()
            ins.op, ins.src, ins.mode, ins.pad = op, src, mode, 0
            if int32:
                ins.imm_i32 = int(imm)
            else:
                ins.imm = float(imm)
            ch.code[i] = ins
        return ch


def compile_chain(chain: LinqChain, element: int = LINQ_ELEMENT_F32, arch: str = "gfx950") -> int:
    """Compiles a program's ToArray kernel with hipRTC (no device needed); returns its code size.
    Raises HipError(DC_ERR_COMPILE) when the generated source does not compile."""
    size = C.c_size_t(0)
    check(load().dc_linq_chain_compile(C.byref(chain), element, arch.encode(), C.byref(size)), "dc_linq_chain_compile")
    return size.value


def can_fault_i32(chain: LinqChain) -> bool:
    """Whether an int32 program can throw (then the _i32 entry points need a fault word)."""
    out = C.c_int32(-1)
    check(load().dc_linq_chain_can_fault_i32(C.byref(chain), C.byref(out)), "dc_linq_chain_can_fault_i32")
    return bool(out.value)


def where_gt0_select_2x_plus_1() -> LinqChain:
    """The benchmark chain ``Where(x => x > 0f).Select(x => x * 2f + 1f)``."""
    return LinqChain.assemble([
        (LOAD, SRC_ELEM, 0.0), (CMP_GT, SRC_IMM, 0.0), (FILTER, SRC_IMM, 0.0),
        (LOAD, SRC_ELEM, 0.0), (MUL, SRC_IMM, 2.0), (ADD, SRC_IMM, 1.0), (MAP, SRC_IMM, 0.0),
    ])


class HipError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {error_string(status)} (status {status})")


_i32, _i64, _u32, _u64, _sz, _P = C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_size_t, C.c_void_p
_PP = C.POINTER(C.c_void_p)

# name -> argtypes (every function returns int32 unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "dc_hip_error_string": [_i32],
    "dc_hip_abi_version": [],
    "dc_hip_device_count": [C.POINTER(_i32)],
    "dc_hip_device_info_get": [_i32, C.POINTER(DeviceInfo)],
    "dc_hip_ctx_create": [_i32, _PP],
    "dc_hip_ctx_destroy": [_P],
    "dc_hip_ctx_device": [_P, C.POINTER(_i32)],
    "dc_hip_synchronize": [_P],
    "dc_hip_malloc": [_P, _sz, _PP],
    "dc_hip_free": [_P, _P],
    "dc_hip_malloc_host": [_P, _sz, _PP],
    "dc_hip_free_host": [_P, _P],
    "dc_hip_memcpy_h2d_async": [_P, _P, _P, _sz],
    "dc_hip_memcpy_d2h_async": [_P, _P, _P, _sz],
    "dc_hip_memcpy_d2d_async": [_P, _P, _P, _sz],
    "dc_hip_memset_async": [_P, _P, _i32, _sz],
    "dc_hip_mem_info": [_P, C.POINTER(_sz), C.POINTER(_sz)],
    "dc_hip_event_create": [_P, _PP],
    "dc_hip_event_destroy": [_P],
    "dc_hip_event_record": [_P, _P],
    "dc_hip_event_synchronize": [_P],
    "dc_hip_event_elapsed_ms": [_P, _P, C.POINTER(C.c_float)],
    "dc_hip_module_load": [_P, C.c_char_p, _PP],
    "dc_hip_module_load_data": [_P, _P, _PP],
    "dc_hip_module_unload": [_P],
    "dc_hip_module_get_function": [_P, C.c_char_p, _PP],
    "dc_hip_launch_kernel": [_P, _P, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _PP],
    "dc_hip_default_module_path": [],
    "dc_hip_fill_uniform_f32": [_P, _P, _i64, _u64, _u32, _i32],
    "dc_hip_fill_uniform_i32": [_P, _P, _i64, _u64, _u32, _i32, _i32],
    "dc_gen_uniform_f32": [_P, _i64, _u64, _u32, _i32],
    "dc_gen_uniform_i32": [_P, _i64, _u64, _u32, _i32, _i32],
    "dc_gen_zipf_csr_rowptr": [_i64, C.c_double, _i32, _u64, _P],
    "dc_gen_zipf_csr_fill": [_i64, _i64, _u64, _P, _P, _P],
    "dc_hip_vector_add_f32": [_P, _P, _P, _P, _i64],
    "dc_hip_reduce_sum_f32": [_P, _P, _i64, _P],
    "dc_hip_reduce_sum_i32": [_P, _P, _i64, _P, _P],
    "dc_linq_chain_validate": [C.POINTER(LinqChain)],
    "dc_hip_linq_where_select_f32": [_P, C.POINTER(LinqChain), _P, _i64, _P, _P],
    "dc_hip_linq_where_select_sum_f32": [_P, C.POINTER(LinqChain), _P, _i64, _P, _P],
    "dc_hip_linq_where_select_sum_f32_noalloc": [_P, C.POINTER(LinqChain), _P, _i64, _P, _P],
    "dc_hip_host_device_pointer": [_P, _P, _P],
    "dc_hip_linq_where_select_minmax_f32": [_P, C.POINTER(LinqChain), _P, _i64, _i32, _P, _P],
    "dc_hip_linq_to_array_strategy": [_P, _P, _i64, _P],
    "dc_linq_chain_can_fault_i32": [C.POINTER(LinqChain), C.POINTER(_i32)],
    "dc_linq_chain_validate_i32": [C.POINTER(LinqChain)],
    "dc_linq_chain_compile": [C.POINTER(LinqChain), _i32, C.c_char_p, C.POINTER(_sz)],
    "dc_hip_linq_compile_stats": [_P, C.POINTER(_i64), C.POINTER(_i64)],
    "dc_hip_linq_where_select_i32": [_P, C.POINTER(LinqChain), _P, _i64, _P, _P, _P],
    "dc_hip_linq_where_select_sum_i32": [_P, C.POINTER(LinqChain), _P, _i64, _P, _P, _P, _P],
    "dc_hip_linq_where_select_minmax_i32": [_P, C.POINTER(LinqChain), _P, _i64, _i32, _P, _P, _P],
    "dc_hip_gemm_f32": [_P, _P, _P, _P, _i64, _i64, _i64],
    "dc_hip_gemm_bf16": [_P, _P, _P, _P, _i64, _i64, _i64],
    "dc_hip_convert_f32_to_bf16": [_P, _P, _P, _i64],
    "dc_hip_spmv_csr_f32": [_P, _P, _P, _P, _P, _P, _i64, _i64, _i64],
    "dc_hip_spmv_csr_f64": [_P, _P, _P, _P, _P, _P, _i64, _i64, _i64],
    "dc_hip_spmv_csr_i32": [_P, _P, _P, _P, _P, _P, _i64, _i64, _i64],
    "dc_hip_spmv_power_iterate_f32": [_P, _P, _P, _P, _P, _P, _i64, _i64, _i32, _P],
    "dc_hip_spmv_plan_create": [_P, _P, _P, _P, _i64, _i64, _i64, _i64, _PP],
    "dc_hip_spmv_plan_execute_f32": [_P, _P, _P, _P],
    "dc_hip_spmv_plan_power_iterate_f32": [_P, _P, _P, _P, _i32, _P],
    "dc_hip_spmv_plan_info": [_P, C.POINTER(_i32), C.POINTER(_i64), C.POINTER(_i64)],
    "dc_hip_spmv_plan_destroy": [_P],
}
_RESTYPES = {"dc_hip_error_string": C.c_char_p, "dc_hip_default_module_path": C.c_char_p}

_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load the HIP library. Raises if it has not been built (no silent fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m dotcompute_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, C.c_int32)
        _lib = L
    return _lib


_bench_lib: C.CDLL | None = None


def load_bench() -> C.CDLL:
    """The measurement-only probe library (dotcompute_amd/probes), loaded after the product library
    whose contexts it runs on."""
    global _bench_lib
    if _bench_lib is None:
        load()
        if not os.path.exists(BENCH_LIB_PATH):
            raise ImportError(f"{BENCH_LIB_PATH} is missing: build it with `python -m dotcompute_amd.build`")
        L = C.CDLL(BENCH_LIB_PATH)
        L.dc_bench_stream_probe.argtypes = [_P, _i32, _P, _P, _i64]
        L.dc_bench_stream_probe.restype = C.c_int32
        _bench_lib = L
    return _bench_lib


def error_string(status: int) -> str:
    return load().dc_hip_error_string(status).decode()


def check(status: int, where: str) -> None:
    if status != DC_OK:
        raise HipError(status, where)


def device_count() -> int:
    c = C.c_int32(0)
    check(load().dc_hip_device_count(C.byref(c)), "dc_hip_device_count")
    return c.value


def device_info(device: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    check(load().dc_hip_device_info_get(device, C.byref(info)), "dc_hip_device_info_get")
    return info


def header_symbols() -> list[str]:
    """Every function the public header declares (used by the ABI tests)."""
    import re

    text = open(HEADER).read()
    return sorted(set(re.findall(r"DC_HIP_API\s+[\w\s\*]+?\b(dc_\w+)\s*\(", text)))


@dataclass
class DeviceArray:
    """A device allocation owned by a Context (freed exactly once)."""

    ctx: "Context"
    ptr: int
    nbytes: int
    dtype: np.dtype
    shape: tuple

    @property
    def size(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    def copy_from(self, host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host, self.dtype)
        assert host.nbytes <= self.nbytes
        check(load().dc_hip_memcpy_h2d_async(self.ctx.handle, self.ptr, host.ctypes.data, host.nbytes), "h2d")
        self.ctx.synchronize()
        return self

    def to_host(self, count: int | None = None) -> np.ndarray:
        n = self.size if count is None else count
        out = np.empty(n, self.dtype)
        if n:
            check(load().dc_hip_memcpy_d2h_async(self.ctx.handle, out.ctypes.data, self.ptr, out.nbytes), "d2h")
            self.ctx.synchronize()
        return out if count is not None else out.reshape(self.shape)

    def free(self) -> None:
        if self.ptr:
            check(load().dc_hip_free(self.ctx.handle, self.ptr), "dc_hip_free")
            self.ptr = 0


class Event:
    def __init__(self, ctx: "Context"):
        self.ctx = ctx
        h = C.c_void_p()
        check(load().dc_hip_event_create(ctx.handle, C.byref(h)), "dc_hip_event_create")
        self.handle = h.value

    def record(self) -> None:
        check(load().dc_hip_event_record(self.ctx.handle, self.handle), "dc_hip_event_record")

    def synchronize(self) -> None:
        check(load().dc_hip_event_synchronize(self.handle), "dc_hip_event_synchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(load().dc_hip_event_elapsed_ms(self.handle, end.handle, C.byref(ms)), "dc_hip_event_elapsed_ms")
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            load().dc_hip_event_destroy(self.handle)
            self.handle = None


class Context:
    """One gfx950 device + stream (dc_hip_ctx)."""

    def __init__(self, device: int = 0):
        L = load()
        h = C.c_void_p()
        check(L.dc_hip_ctx_create(device, C.byref(h)), f"dc_hip_ctx_create({device})")
        self.handle = h.value
        self.device = device
        self._arrays: list[DeviceArray] = []

    # ---- lifetime ----
    def close(self) -> None:
        if self.handle:
            for a in self._arrays:
                a.free()
            check(load().dc_hip_ctx_destroy(self.handle), "dc_hip_ctx_destroy")
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def synchronize(self) -> None:
        check(load().dc_hip_synchronize(self.handle), "dc_hip_synchronize")

    # ---- memory ----
    def empty(self, shape, dtype) -> DeviceArray:
        shape = (shape,) if isinstance(shape, (int, np.integer)) else tuple(shape)
        dtype = np.dtype(dtype)
        nbytes = int(np.prod(shape)) * dtype.itemsize if shape else dtype.itemsize
        p = C.c_void_p()
        check(load().dc_hip_malloc(self.handle, max(nbytes, 1), C.byref(p)), f"dc_hip_malloc({nbytes})")
        arr = DeviceArray(self, p.value, nbytes, dtype, shape)
        self._arrays.append(arr)
        return arr

    def to_device(self, host: np.ndarray) -> DeviceArray:
        host = np.ascontiguousarray(host)
        return self.empty(host.shape, host.dtype).copy_from(host)

    def event(self) -> Event:
        return Event(self)

    def free(self, arr: DeviceArray) -> None:
        arr.free()
        self._arrays = [a for a in self._arrays if a is not arr]

    # ---- generators ----
    def fill_uniform_f32(self, arr: DeviceArray, seed: int, stream: int = 0, unit_interval: bool = False) -> None:
        check(load().dc_hip_fill_uniform_f32(self.handle, arr.ptr, arr.size, seed, stream, int(unit_interval)), "fill_f32")

    def fill_uniform_i32(self, arr: DeviceArray, seed: int, stream: int = 1, lo: int = -1000, hi: int = 1000) -> None:
        check(load().dc_hip_fill_uniform_i32(self.handle, arr.ptr, arr.size, seed, stream, lo, hi), "fill_i32")

    # ---- ops (enqueue only; results on device) ----
    def vector_add_f32(self, a: DeviceArray, b: DeviceArray, r: DeviceArray, n: int | None = None) -> None:
        n = r.size if n is None else n
        check(load().dc_hip_vector_add_f32(self.handle, a.ptr, b.ptr, r.ptr, n), "dc_hip_vector_add_f32")

    def stream_probe(self, kind: int, src: DeviceArray, dst: DeviceArray, n: int) -> None:
        """Measurement-only streaming probe (PROBE_COPY / PROBE_READ2_WRITE1 / PROBE_READ), from the
        separate probe library."""
        check(load_bench().dc_bench_stream_probe(self.handle, kind, src.ptr, dst.ptr, n), "dc_bench_stream_probe")

    def reduce_sum_f32(self, x: DeviceArray, out: DeviceArray, n: int | None = None) -> None:
        n = x.size if n is None else n
        check(load().dc_hip_reduce_sum_f32(self.handle, x.ptr, n, out.ptr), "dc_hip_reduce_sum_f32")

    def reduce_sum_i32(self, x: DeviceArray, out: DeviceArray, overflow: DeviceArray | None, n: int | None = None) -> None:
        n = x.size if n is None else n
        check(load().dc_hip_reduce_sum_i32(self.handle, x.ptr, n, out.ptr, overflow.ptr if overflow else None),
              "dc_hip_reduce_sum_i32")

    def where_select_f32(self, chain: LinqChain, x: DeviceArray, out: DeviceArray, count: DeviceArray,
                         n: int | None = None) -> None:
        n = x.size if n is None else n
        check(load().dc_hip_linq_where_select_f32(self.handle, C.byref(chain), x.ptr, n, out.ptr, count.ptr),
              "dc_hip_linq_where_select_f32")

    def compile_stats(self) -> tuple[int, int]:
        """(launches of run-time compiled LINQ kernels on this context, failed compilations)."""
        a, b = C.c_int64(0), C.c_int64(0)
        check(load().dc_hip_linq_compile_stats(self.handle, C.byref(a), C.byref(b)), "dc_hip_linq_compile_stats")
        return a.value, b.value

    def to_array_strategy(self, x: DeviceArray, n: int | None = None) -> int:
        """Kernel that where_select_f32 uses for this input: STRATEGY_LOOKBACK or STRATEGY_ROUNDS."""
        n = x.size if n is None else n
        out = C.c_int32(-1)
        check(load().dc_hip_linq_to_array_strategy(self.handle, x.ptr, n, C.byref(out)),
              "dc_hip_linq_to_array_strategy")
        return out.value

    def where_select_sum_f32(self, chain: LinqChain, x: DeviceArray, sum_out: DeviceArray | None,
                             count: DeviceArray | None, n: int | None = None) -> None:
        n = x.size if n is None else n
        check(load().dc_hip_linq_where_select_sum_f32(self.handle, C.byref(chain), x.ptr, n,
                                                     sum_out.ptr if sum_out else None,
                                                     count.ptr if count else None),
              "dc_hip_linq_where_select_sum_f32")

    def where_select_minmax_f32(self, chain: LinqChain, x: DeviceArray, op: int, value_out: DeviceArray | None,
                                count: DeviceArray | None, n: int | None = None) -> None:
        """op = LINQ_MIN, LINQ_MAX, LINQ_FOLD_MIN or LINQ_FOLD_MAX; value_out: float32[1], count:
        int64[1] (device)."""
        n = x.size if n is None else n
        check(load().dc_hip_linq_where_select_minmax_f32(self.handle, C.byref(chain), x.ptr, n, op,
                                                        value_out.ptr if value_out else None,
                                                        count.ptr if count else None),
              "dc_hip_linq_where_select_minmax_f32")

    # ---- int32 chains (C# int semantics); fault: int64[1] (device) or None for programs that cannot throw
    def where_select_i32(self, chain: LinqChain, x: DeviceArray, out: DeviceArray, count: DeviceArray,
                         fault: DeviceArray | None, n: int | None = None) -> None:
        n = x.size if n is None else n
        check(load().dc_hip_linq_where_select_i32(self.handle, C.byref(chain), x.ptr, n, out.ptr, count.ptr,
                                                 fault.ptr if fault else None), "dc_hip_linq_where_select_i32")

    def where_select_sum_i32(self, chain: LinqChain, x: DeviceArray, sum_out: DeviceArray | None,
                             count: DeviceArray | None, overflow: DeviceArray | None, fault: DeviceArray | None,
                             n: int | None = None) -> None:
        n = x.size if n is None else n
        check(load().dc_hip_linq_where_select_sum_i32(self.handle, C.byref(chain), x.ptr, n,
                                                     sum_out.ptr if sum_out else None, count.ptr if count else None,
                                                     overflow.ptr if overflow else None, fault.ptr if fault else None),
              "dc_hip_linq_where_select_sum_i32")

    def where_select_minmax_i32(self, chain: LinqChain, x: DeviceArray, op: int, value_out: DeviceArray | None,
                                count: DeviceArray | None, fault: DeviceArray | None, n: int | None = None) -> None:
        n = x.size if n is None else n
        check(load().dc_hip_linq_where_select_minmax_i32(self.handle, C.byref(chain), x.ptr, n, op,
                                                        value_out.ptr if value_out else None,
                                                        count.ptr if count else None, fault.ptr if fault else None),
              "dc_hip_linq_where_select_minmax_i32")

    def gemm_f32(self, a: DeviceArray, b: DeviceArray, c: DeviceArray, m: int, n: int, k: int) -> None:
        check(load().dc_hip_gemm_f32(self.handle, a.ptr, b.ptr, c.ptr, m, n, k), "dc_hip_gemm_f32")

    def gemm_bf16(self, a: DeviceArray, b: DeviceArray, c: DeviceArray, m: int, n: int, k: int) -> None:
        check(load().dc_hip_gemm_bf16(self.handle, a.ptr, b.ptr, c.ptr, m, n, k), "dc_hip_gemm_bf16")

    def convert_f32_to_bf16(self, x: DeviceArray, out: DeviceArray, n: int | None = None) -> None:
        n = x.size if n is None else n
        check(load().dc_hip_convert_f32_to_bf16(self.handle, x.ptr, out.ptr, n), "dc_hip_convert_f32_to_bf16")

    def spmv_csr_f32(self, rp: DeviceArray, col: DeviceArray, val: DeviceArray, x: DeviceArray, y: DeviceArray,
                     rows: int, cols: int, nnz: int) -> None:
        check(load().dc_hip_spmv_csr_f32(self.handle, rp.ptr, col.ptr, val.ptr, x.ptr, y.ptr, rows, cols, nnz),
              "dc_hip_spmv_csr_f32")

    def spmv_csr(self, rp: DeviceArray, col: DeviceArray, val: DeviceArray, x: DeviceArray, y: DeviceArray,
                 rows: int, cols: int, nnz: int) -> None:
        """y = A·x for float32, float64 or int32 values (the element type of `val`)."""
        name = {np.dtype(np.float32): "dc_hip_spmv_csr_f32", np.dtype(np.float64): "dc_hip_spmv_csr_f64",
                np.dtype(np.int32): "dc_hip_spmv_csr_i32"}[np.dtype(val.dtype)]
        check(getattr(load(), name)(self.handle, rp.ptr, col.ptr, val.ptr, x.ptr, y.ptr, rows, cols, nnz), name)

    def spmv_power_iterate_f32(self, rp, col, val, x, y, rows: int, nnz: int, iterations: int,
                               last_sum: DeviceArray | None = None) -> None:
        check(load().dc_hip_spmv_power_iterate_f32(self.handle, rp.ptr, col.ptr, val.ptr, x.ptr, y.ptr, rows, nnz,
                                                  iterations, last_sum.ptr if last_sum else None),
              "dc_hip_spmv_power_iterate_f32")

    def spmv_plan(self, rp: DeviceArray, col: DeviceArray, val: DeviceArray, rows: int, cols: int, nnz: int,
                  slice_cols_max: int = 0) -> "SpmvPlan":
        h = C.c_void_p()
        check(load().dc_hip_spmv_plan_create(self.handle, rp.ptr, col.ptr, val.ptr, rows, cols, nnz, slice_cols_max,
                                             C.byref(h)), "dc_hip_spmv_plan_create")
        return SpmvPlan(self, h.value, rows, cols)


class SpmvPlan:
    """Tiled SpMV plan (dc_hip_spmv_plan_*): built once, executed many times."""

    def __init__(self, ctx: "Context", handle, rows: int, cols: int):
        self.ctx, self.handle, self.rows, self.cols = ctx, handle, rows, cols

    def info(self) -> tuple[int, int, int]:
        s, w, b = C.c_int32(), C.c_int64(), C.c_int64()
        check(load().dc_hip_spmv_plan_info(self.handle, C.byref(s), C.byref(w), C.byref(b)), "dc_hip_spmv_plan_info")
        return s.value, w.value, b.value

    def execute(self, x: DeviceArray, y: DeviceArray) -> None:
        check(load().dc_hip_spmv_plan_execute_f32(self.ctx.handle, self.handle, x.ptr, y.ptr),
              "dc_hip_spmv_plan_execute_f32")

    def power_iterate(self, x: DeviceArray, y: DeviceArray, iterations: int, last_sum: DeviceArray | None = None) -> None:
        check(load().dc_hip_spmv_plan_power_iterate_f32(self.ctx.handle, self.handle, x.ptr, y.ptr, iterations,
                                                        last_sum.ptr if last_sum else None),
              "dc_hip_spmv_plan_power_iterate_f32")

    def destroy(self) -> None:
        if self.handle:
            check(load().dc_hip_spmv_plan_destroy(self.handle), "dc_hip_spmv_plan_destroy")
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


def gen_zipf_csr(rows: int, seed: int, alpha: float = 2.0, max_degree: int = 4096, cols: int | None = None):
    """Host-side synthetic PageRank graph (product generator, multithreaded C++)."""
    L = load()
    cols = rows if cols is None else cols
    rp = np.empty(rows + 1, np.int32)
    check(L.dc_gen_zipf_csr_rowptr(rows, alpha, max_degree, seed, rp.ctypes.data), "dc_gen_zipf_csr_rowptr")
    nnz = int(rp[-1])
    col = np.empty(nnz, np.int32)
    val = np.empty(nnz, np.float32)
    check(L.dc_gen_zipf_csr_fill(rows, cols, seed, rp.ctypes.data, col.ctypes.data, val.ctypes.data),
          "dc_gen_zipf_csr_fill")
    return rp, col, val


def gen_uniform_f32(n: int, seed: int, stream: int = 0, unit_interval: bool = False) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(load().dc_gen_uniform_f32(out.ctypes.data, n, seed, stream, int(unit_interval)), "dc_gen_uniform_f32")
    return out


def gen_uniform_i32(n: int, seed: int, stream: int = 1, lo: int = -1000, hi: int = 1000) -> np.ndarray:
    out = np.empty(n, np.int32)
    check(load().dc_gen_uniform_i32(out.ctypes.data, n, seed, stream, lo, hi), "dc_gen_uniform_i32")
    return out
