"""Run-time compilation of LINQ programs without a device: the generated kernel source compiles with
hipRTC for gfx950 for programs over every instruction (float32 and int32, with and without the save
registers), and bad requests are refused. The GPU tests (test_gpu_linq_compiled.py) check what the
compiled kernels compute."""
import pytest

from dotcompute_amd import hip
from dotcompute_amd.hip import (ABS, ADD, CEIL, CMP_AND, CMP_EQ, CMP_GT, CMP_LT, CMP_OR, DIV, FILTER, FLOOR, LOAD,
                                MAP, MAX, MIN, MUL, NEG, PAND_Q, PNOT, POR_Q, POW, PSTORE, RDIV, REM, ROUND, RPOW,
                                RREM, RSUB, SQRT, SRC_ELEM, SRC_IMM, SRC_S0, SRC_S1, STORE_S0, STORE_S1, SUB,
                                LinqChain)

try:
    hip.load()
    HAVE_LIB = True
except ImportError:
    HAVE_LIB = False

needs_lib = pytest.mark.skipif(not HAVE_LIB, reason="libdotcompute_hip.so is not built")

EVERY_FLOAT_OP = [(LOAD, SRC_ELEM, 0), (STORE_S0, SRC_IMM, 0), (ADD, SRC_IMM, 1.5), (SUB, SRC_S0, 0),
                  (RSUB, SRC_IMM, 2), (MUL, SRC_ELEM, 0), (DIV, SRC_IMM, 3), (RDIV, SRC_IMM, 5), (REM, SRC_IMM, 0.75),
                  (RREM, SRC_IMM, 9), (MIN, SRC_IMM, 4), (MAX, SRC_S0, 0), (NEG, SRC_IMM, 0), (ABS, SRC_IMM, 0),
                  (SQRT, SRC_IMM, 0), (FLOOR, SRC_IMM, 0), (CEIL, SRC_IMM, 0), (ROUND, SRC_IMM, 0),
                  (POW, SRC_IMM, 1.5), (RPOW, SRC_S0, 0), (STORE_S1, SRC_IMM, 0), (CMP_GT, SRC_S1, 0), (PSTORE, SRC_IMM, 0), (CMP_LT, SRC_IMM, 3, CMP_AND),
                  (CMP_EQ, SRC_IMM, 0, CMP_OR), (PAND_Q, SRC_IMM, 0), (POR_Q, SRC_IMM, 0), (PNOT, SRC_IMM, 0),
                  (FILTER, SRC_IMM, 0), (MAP, SRC_IMM, 0)]
EVERY_INT_OP = [(LOAD, SRC_ELEM, 0), (STORE_S0, SRC_IMM, 0), (ADD, SRC_IMM, 7), (SUB, SRC_S0, 0), (RSUB, SRC_IMM, 2),
                (MUL, SRC_ELEM, 0), (DIV, SRC_IMM, 3), (DIV, SRC_IMM, -7), (DIV, SRC_ELEM, 0), (REM, SRC_IMM, 2),
                (REM, SRC_IMM, -1), (RDIV, SRC_IMM, 100), (RREM, SRC_IMM, 9), (MIN, SRC_IMM, 4), (MAX, SRC_S0, 0),
                (NEG, SRC_IMM, 0), (ABS, SRC_IMM, 0), (STORE_S1, SRC_IMM, 0), (CMP_GT, SRC_S1, 0), (FILTER, SRC_IMM, 0),
                (MAP, SRC_IMM, 0)]


@needs_lib
def test_every_float_instruction_compiles():
    assert hip.compile_chain(LinqChain.assemble(EVERY_FLOAT_OP), hip.LINQ_ELEMENT_F32) > 0


@needs_lib
def test_every_int_instruction_compiles():
    assert hip.compile_chain(LinqChain.assemble(EVERY_INT_OP, int32=True), hip.LINQ_ELEMENT_I32) > 0


@needs_lib
def test_short_programs_compile():
    sq = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (MUL, SRC_ELEM, 0), (MAP, SRC_IMM, 0)])
    assert hip.compile_chain(sq) > 0
    assert hip.compile_chain(LinqChain.assemble([], int32=True), hip.LINQ_ELEMENT_I32) > 0  # the identity


@needs_lib
def test_bad_requests_are_refused():
    sq = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (SQRT, SRC_IMM, 0), (MAP, SRC_IMM, 0)], int32=True)
    with pytest.raises(hip.HipError) as e:
        hip.compile_chain(sq, hip.LINQ_ELEMENT_I32)  # no int32 square root
    assert e.value.status == hip.DC_ERR_UNSUPPORTED
    with pytest.raises(hip.HipError) as e:
        hip.compile_chain(LinqChain.assemble([(40, SRC_IMM, 0)]))
    assert e.value.status == hip.DC_ERR_UNSUPPORTED
    with pytest.raises(hip.HipError) as e:
        hip.compile_chain(LinqChain.assemble([]), 7)
    assert e.value.status == hip.DC_ERR_INVALID_ARGUMENT
