"""Emits gfx950 HIP kernels and the C++ kernel registry for [Kernel] methods.

Execution model of an emitted kernel: the reference's CPU invoker, run one work item per GPU
thread. The orchestrator launches ceil(work / 256) workgroups of 256 threads over the flat range
[0, work) (work = the first writable buffer's length, KernelExecutionService.cs:382-406); each
thread rebuilds the work item's coordinates from the trailing integer parameters exactly as the
generated CPU invoker does (KernelExecutionMetadataEmitter.cs:203-245) and maps the KernelContext
intrinsics the same way (ThreadId -> coordinate, BlockDim -> extent, BlockId -> 0, GridDim -> 1,
CpuInvokerBodyRewriter :458-495). So a body computes on the GPU what it computes on the reference's
CPU backend, whichever way it spells its index, and the generated CUDA's per-block threadIdx
meaning (:442) does not arise.

C# semantics kept by the emitted code:
  - span accesses are bounds-checked: an index outside [0, Length) sets the launch's
    IndexOutOfRange word (the host throws IndexOutOfRangeException) and the access is dropped;
  - `.Length` is each buffer's own length;
  - integer arithmetic wraps (the library is built with -fwrapv), shift counts are masked to the
    operand width, integer division or remainder by zero raises DivideByZeroException and
    MinValue / -1 raises OverflowException;
  - every float operation rounds once (no contraction), float -> integer casts saturate and map
    NaN to 0 (.NET 9 and later), Math.Min/Max follow the IEEE 754-2019 minimum/maximum that
    .NET implements (NaN wins, -0 < +0).
"""
from __future__ import annotations

from . import csharp as cs
from .csharp import (Assign, Binary, Block, BoolLit, Break, Call, Cast, Cond, Continue, ExprStmt, For, If, Index,
                     Intrinsic, KernelMethod, Length, Lit, LocalDecl, Name, Return, Unary, Unsupported, While)

CTYPE = {"float": "float", "double": "double", "int": "int32_t", "uint": "uint32_t", "long": "int64_t",
         "ulong": "uint64_t", "short": "int16_t", "ushort": "uint16_t", "byte": "uint8_t", "sbyte": "int8_t",
         "bool": "bool", "char": "uint16_t"}
CXX_KEYWORDS = {"auto", "register", "template", "typename", "signed", "unsigned", "union", "friend", "inline",
                "mutable", "export", "delete", "not", "and", "or", "xor", "bitand", "bitor", "compl", "not_eq",
                "and_eq", "or_eq", "xor_eq", "asm", "typeid", "dynamic_cast", "reinterpret_cast", "static_cast",
                "const_cast", "constexpr", "decltype", "noexcept", "nullptr", "thread_local", "alignas", "alignof",
                "char16_t", "char32_t", "static_assert", "concept", "requires", "co_await", "co_return",
                "co_yield", "wchar_t", "int8_t", "int16_t", "int32_t", "int64_t", "uint8_t", "uint16_t",
                "uint32_t", "uint64_t", "min", "max", "sqrt", "sqrtf", "fabs", "fabsf", "dcg", "threadIdx",
                "blockIdx", "blockDim", "gridDim"}

BLOCK = 256
SMALL_INTS = ("sbyte", "byte", "short", "ushort", "char")


def ident(name: str) -> str:
    name = name.lstrip("@")
    if name.startswith("__"):
        raise Unsupported(f"identifier {name} (names starting with __ are reserved for the generator)")
    return name + "_" if name in CXX_KEYWORDS else name


class KernelEmitter:
    def __init__(self, km: KernelMethod, checker: cs.Checker):
        self.km = km
        self.c = checker
        self.buf_index = {p.name: i for i, p in enumerate(q for q in km.params if q.is_buffer)}
        self.tmp = 0

    # ---- expressions -----------------------------------------------------------------------
    def conv(self, e, to: str) -> str:
        s = self.ex(e)
        if e.ty == to:
            return s
        if to in cs.INTEGRAL and e.ty in cs.FLOATING:
            raise Unsupported("implicit floating -> integer conversion")
        return f"(({CTYPE[to]})({s}))"

    def ex(self, e) -> str:
        if isinstance(e, Lit):
            ty, digits = cs.literal_type(e.text)
            if ty in ("float", "double"):
                d = digits if ("." in digits or "e" in digits.lower()) else digits + ".0"
                if d.startswith("."):
                    d = "0" + d
                return d + ("f" if ty == "float" else "")
            return digits + {"int": "", "uint": "u", "long": "ll", "ulong": "ull"}[ty]
        if isinstance(e, BoolLit):
            return "true" if e.value else "false"
        if isinstance(e, Name):
            return ident(e.ident)
        if isinstance(e, Intrinsic):
            ax = e.axis.lower()
            return {"ThreadId": f"__{ax}", "BlockDim": f"__{ax}ext", "BlockId": "0", "GridDim": "1"}[e.kind]
        if isinstance(e, Length):
            return f"((int32_t)__len{self.buf_index[e.buffer]})"
        if isinstance(e, Index):
            k = self.buf_index[e.buffer]
            return f"dcg::ld({ident(e.buffer)}, (int64_t)({self.ex(e.index)}), __len{k}, __l)"
        if isinstance(e, Cast):
            src = e.expr.ty
            if e.to == src:
                return f"({self.ex(e.expr)})"
            if src in cs.FLOATING and e.to in cs.INTEGRAL:
                if e.to in SMALL_INTS:
                    raise Unsupported(f"cast from {src} to {e.to}")
                return f"dcg::f2i<{CTYPE[e.to]}>({self.ex(e.expr)})"
            return f"(({CTYPE[e.to]})({self.ex(e.expr)}))"
        if isinstance(e, Call):
            fname = e.func.split(".")[1]
            if e.func.startswith("MathF."):
                args = [self.conv(a, "float") for a in e.args]
                ty = "float"
            elif fname == "Sqrt":
                args = [self.conv(e.args[0], "double")]
                ty = "double"
            else:
                ty = e.ty
                args = [self.conv(a, ty) for a in e.args]
            if fname == "Sqrt":
                return f"{'sqrtf' if ty == 'float' else 'sqrt'}({args[0]})"
            if fname == "Abs":
                if ty in cs.FLOATING:
                    return f"{'fabsf' if ty == 'float' else 'fabs'}({args[0]})"
                return f"dcg::abs_checked<{CTYPE[ty]}>({args[0]}, __l)"
            fn = "min" if fname == "Min" else "max"
            if ty in cs.FLOATING:
                return f"dcg::f{fn}_net<{CTYPE[ty]}>({args[0]}, {args[1]})"
            return f"dcg::i{fn}<{CTYPE[ty]}>({args[0]}, {args[1]})"
        if isinstance(e, Unary):
            if e.op in ("++", "--"):
                if not isinstance(e.expr, Name):
                    raise Unsupported("++/-- of a buffer element inside an expression")
                n = ident(e.expr.ident)
                return f"({n}{e.op})" if e.postfix else f"({e.op}{n})"
            if e.op == "!":
                return f"(!{self.ex(e.expr)})"
            return f"({e.op}{self.conv(e.expr, e.ty)})"
        if isinstance(e, Binary):
            return self.binary(e.op, e.left, e.right, e.operand_ty, e.ty)
        if isinstance(e, Cond):
            return f"({self.ex(e.cond)} ? {self.conv(e.a, e.ty)} : {self.conv(e.b, e.ty)})"
        if isinstance(e, Assign):
            if not isinstance(e.target, Name):
                raise Unsupported("buffer element assignment inside an expression")
            n = ident(e.target.ident)
            return f"({n} = {self.assigned_value(e, n)})"
        raise Unsupported(f"expression {type(e).__name__}")

    def binary(self, op: str, left, right, p: str, result: str, left_text: str | None = None) -> str:
        lt = left_text if left_text is not None else None

        def L():
            if lt is not None:
                return lt if left.ty == p else f"(({CTYPE[p]})({lt}))"
            return self.conv(left, p)

        if op in ("&&", "||"):
            return f"({self.ex(left)} {op} {self.ex(right)})"
        if p == "bool":
            return f"((bool)({L()} {op} {self.ex(right)}))"
        if op in ("<<", ">>"):
            fn = "shl" if op == "<<" else "shr"
            return f"dcg::{fn}<{CTYPE[p]}>({L()}, (int32_t)({self.ex(right)}))"
        r = self.conv(right, p)
        if op in ("/", "%") and p in cs.INTEGRAL:
            fn = "idiv" if op == "/" else "irem"
            return f"dcg::{fn}<{CTYPE[p]}>({L()}, {r}, __l)"
        if op == "%":  # floating remainder: truncated, like C's fmod (C# 12.10.4)
            return f"{'fmodf' if p == 'float' else 'fmod'}({L()}, {r})"
        return f"({L()} {op} {r})"

    def assigned_value(self, a: Assign, target_text: str) -> str:
        """Value stored by `target op= value`, converted to the target's type."""
        tt = a.target.ty if isinstance(a.target, Name) else a.ty
        if a.op == "=":
            return self.conv(a.value, tt)
        op = a.op[:-1]
        fake_left = Name("__target")
        fake_left.ty = tt
        v = self.binary(op, fake_left, a.value, a.operand_ty, a.operand_ty, left_text=target_text)
        return v if a.operand_ty == tt else f"(({CTYPE[tt]})({v}))"

    @staticmethod
    def cond(text: str) -> str:
        """`(text)` for an if/while/for condition without doubling a pair that already encloses it."""
        if text.startswith("(") and text.endswith(")"):
            depth = 0
            for i, ch in enumerate(text):
                depth += ch == "("
                depth -= ch == ")"
                if depth == 0 and i < len(text) - 1:
                    break
            else:
                return text
        return f"({text})"

    # ---- statements ------------------------------------------------------------------------
    def st(self, s, ind: str, out: list) -> None:
        if isinstance(s, Block):
            out.append(ind + "{")
            for x in s.body:
                self.st(x, ind + "  ", out)
            out.append(ind + "}")
        elif isinstance(s, LocalDecl):
            for name, init in s.names:
                v = self.conv(init, s.ty) if init is not None else f"{CTYPE[s.ty]}()"
                out.append(f"{ind}{CTYPE[s.ty]} {ident(name)} = {v};")
        elif isinstance(s, ExprStmt):
            self.expr_stmt(s.expr, ind, out)
        elif isinstance(s, If):
            out.append(f"{ind}if {self.cond(self.ex(s.cond))}")
            self.st(s.then if isinstance(s.then, Block) else Block([s.then]), ind, out)
            if s.other is not None:
                out.append(f"{ind}else")
                self.st(s.other if isinstance(s.other, Block) else Block([s.other]), ind, out)
        elif isinstance(s, Return):
            out.append(f"{ind}return;")
        elif isinstance(s, Break):
            out.append(f"{ind}break;")
        elif isinstance(s, Continue):
            out.append(f"{ind}continue;")
        elif isinstance(s, For):
            init = ""
            if s.init and isinstance(s.init[0], LocalDecl):
                d = s.init[0]
                init = f"{CTYPE[d.ty]} " + ", ".join(
                    f"{ident(n)} = {self.conv(i, d.ty) if i is not None else CTYPE[d.ty] + '()'}" for n, i in d.names)
            elif s.init:
                init = ", ".join(self.ex(x.expr) for x in s.init)
            cond = self.cond(self.ex(s.cond))[1:-1] if s.cond is not None else ""
            for it in s.iters:
                if isinstance(it, Assign) and isinstance(it.target, Index) or \
                        isinstance(it, Unary) and isinstance(it.expr, Index):
                    raise Unsupported("buffer element update in a for iterator")
            iters = ", ".join(self.ex(x) for x in s.iters)
            out.append(f"{ind}for ({init}; {cond}; {iters})")
            self.st(s.body if isinstance(s.body, Block) else Block([s.body]), ind, out)
        elif isinstance(s, While):
            out.append(f"{ind}while {self.cond(self.ex(s.cond))}")
            self.st(s.body if isinstance(s.body, Block) else Block([s.body]), ind, out)
        else:
            raise Unsupported(f"statement {type(s).__name__}")

    def expr_stmt(self, e, ind: str, out: list) -> None:
        target = None
        if isinstance(e, Assign) and isinstance(e.target, Index):
            target = e.target
        elif isinstance(e, Unary) and e.op in ("++", "--") and isinstance(e.expr, Index):
            target = e.expr
        if target is None:
            out.append(f"{ind}{self.ex(e)};")
            return
        k = self.buf_index[target.buffer]
        buf = ident(target.buffer)
        et = self.c.buffers[target.buffer].element
        self.tmp += 1
        kv = f"__k{self.tmp}"
        elem = f"{buf}[{kv}]"
        out.append(f"{ind}{{")
        out.append(f"{ind}  const int64_t {kv} = (int64_t)({self.ex(target.index)});")
        if isinstance(e, Assign) and e.op == "=":
            vv = f"__v{self.tmp}"
            out.append(f"{ind}  const {CTYPE[et]} {vv} = {self.conv(e.value, et)};")
            out.append(f"{ind}  if ((uint64_t){kv} < (uint64_t)__len{k}) {elem} = {vv};")
        else:
            if isinstance(e, Unary):
                one = Lit("1")
                one.ty = "int"
                a = Assign("+=" if e.op == "++" else "-=", target, one)
                a.ty = et
                a.operand_ty = cs.promote_binary(et, "int")
            else:
                a = e
            out.append(f"{ind}  if ((uint64_t){kv} < (uint64_t)__len{k}) {elem} = {self.assigned_value(a, elem)};")
        out.append(f"{ind}  else dcg::raise(__l, DC_GEN_ERR_INDEX);")
        out.append(f"{ind}}}")

    # ---- kernel ----------------------------------------------------------------------------
    def kernel(self, entry: str) -> str:
        km = self.km
        sig = []
        for p in km.params:
            if p.is_buffer:
                sig.append(f"{'const ' if p.read_only else ''}{CTYPE[p.element]}* {ident(p.name)}")
            else:
                sig.append(f"{CTYPE[p.element]} {ident(p.name)}")
        sig.append("const dc_gen_launch __l")
        lines = [f"// [Kernel] {km.full_name} ({', '.join(km.backends)}): generated from the C# body, line {km.line}",
                 f'extern "C" __global__ __launch_bounds__({BLOCK}) void {entry}({", ".join(sig)}) {{',
                 f"  const int64_t __i = (int64_t)blockIdx.x * {BLOCK} + threadIdx.x;",
                 "  if (__i >= __l.work) return;",
                 "  const int32_t __ii = (int32_t)__i;"]
        ints = [p for p in km.params if not p.is_buffer and p.element in ("int", "uint", "long", "ulong", "short",
                                                                           "ushort", "byte", "sbyte")]
        d = self.c.dims
        if d >= 3 and len(ints) >= 3:
            x, y, z = (f"(int32_t){ident(ints[-k].name)}" for k in (1, 2, 3))
            lines += [f"  const int32_t __xext = {x}, __yext = {y}, __zext = {z};",
                      "  const int32_t __x = __ii % __xext, __y = (__ii / __xext) % __yext, "
                      "__z = __ii / (int32_t)(__xext * __yext);"]
        elif d >= 2 and len(ints) >= 2:
            x, y = (f"(int32_t){ident(ints[-k].name)}" for k in (1, 2))
            lines += [f"  const int32_t __xext = {x}, __yext = {y}, __zext = 1;",
                      "  const int32_t __x = __ii % __xext, __y = __ii / __xext, __z = 0;"]
        else:
            x = f"(int32_t){ident(ints[-1].name)}" if ints else "(int32_t)__l.work"
            lines += [f"  const int32_t __xext = {x}, __yext = 1, __zext = 1;",
                      "  const int32_t __x = __ii, __y = 0, __z = 0;"]
        lines.append("  (void)__xext; (void)__yext; (void)__zext; (void)__x; (void)__y; (void)__z;")
        for name, k in self.buf_index.items():
            lines.append(f"  const int64_t __len{k} = __l.len[{k}]; (void)__len{k};")
        body: list[str] = []
        for s in km.body.body:
            self.st(s, "  ", body)
        lines += body
        lines.append("}")
        return "\n".join(lines)


def _is_work_index(e, idx_names: set) -> bool:
    return (isinstance(e, cs.Intrinsic) and e.kind == "ThreadId" and e.axis == "X") or \
        (isinstance(e, cs.Name) and e.ident in idx_names)


def _walk(node):
    """Every statement and expression node under `node`."""
    yield node
    if isinstance(node, list):
        for x in node:
            yield from _walk(x)
        return
    for v in getattr(node, "__dict__", {}).values():
        if isinstance(v, (cs.Stmt, cs.Expr, list)):
            yield from _walk(v)
        elif isinstance(v, tuple):
            for x in v:
                if isinstance(x, (cs.Stmt, cs.Expr, list)):
                    yield from _walk(x)


def covered_buffers(km: KernelMethod, dims: int) -> set:
    """Buffers whose every element the body writes: a 1-D kernel whose work size is the buffer's
    length (the orchestrator sizes the work by the first writable span) and whose body assigns
    `buf[i] = ...` as an unconditional top-level statement, i being KernelContext.ThreadId.X or a
    local initialised from it and never assigned again, optionally under `if (i < buf.Length)` with
    no else, and with no `return` before it. Such a buffer need not be copied to the device before
    the launch: nothing of its old contents can come back. Every other written buffer is copied in,
    as the reference copies every array (KernelExecutionService.cs:755-763)."""
    if dims != 1:
        return set()
    writable = [p for p in km.params if p.is_buffer and not p.read_only]
    if not writable:
        return set()
    w = writable[0].name
    body = km.body.body
    idx_names = set()
    for s in body:
        if isinstance(s, cs.LocalDecl):
            for name, init in s.names:
                if init is not None and _is_work_index(init, set()):
                    idx_names.add(name)
    for node in _walk(body):  # an index variable assigned again is no longer the work index
        if isinstance(node, cs.Assign) and isinstance(node.target, cs.Name):
            idx_names.discard(node.target.ident)
        if isinstance(node, cs.Unary) and node.op in ("++", "--") and isinstance(node.expr, cs.Name):
            idx_names.discard(node.expr.ident)

    def is_full_write(st) -> bool:
        return isinstance(st, cs.ExprStmt) and isinstance(st.expr, cs.Assign) and st.expr.op == "=" and \
            isinstance(st.expr.target, cs.Index) and st.expr.target.buffer == w and \
            _is_work_index(st.expr.target.index, idx_names)

    def has_return(st) -> bool:
        return any(isinstance(n, cs.Return) for n in _walk(st))

    def first_write(stmts) -> bool:
        for st in stmts:
            if is_full_write(st):
                return True
            if has_return(st):
                return False
        return False

    for st in body:
        if is_full_write(st):
            return {w}
        if isinstance(st, cs.If) and st.other is None and isinstance(st.cond, cs.Binary) and st.cond.op == "<" and \
                _is_work_index(st.cond.left, idx_names) and isinstance(st.cond.right, cs.Length) and \
                st.cond.right.buffer == w:
            inner = st.then.body if isinstance(st.then, cs.Block) else [st.then]
            if first_write(inner):
                return {w}
        if has_return(st):
            return set()
    return set()


def translate(km: KernelMethod, entry: str) -> dict:
    """Returns the registry record of one kernel, with HIP source when the body is translatable."""
    info = {"km": km, "entry": None, "source": None, "dims": 1, "needs_length": False, "reads": set(),
            "writes": set(), "covered": set(), "error": km.error}
    if km.error:  # its parameter list is already outside the subset
        return info
    try:
        checker = cs.analyse(km)
        info["dims"] = checker.dims
        info["needs_length"] = checker.uses_length
        info["reads"] = checker.reads
        info["writes"] = checker.writes
        info["covered"] = covered_buffers(km, checker.dims)
        info["source"] = KernelEmitter(km, checker).kernel(entry)
        info["entry"] = entry
    except Unsupported as e:
        info["error"] = str(e)
        km.error = str(e)
    return info


ELEMENT_TYPE = {"float": "Float32", "double": "Float64", "int": "Int32", "uint": "UInt32", "long": "Int64",
                "ulong": "UInt64", "short": "Int16", "ushort": "UInt16", "byte": "UInt8", "sbyte": "Int8",
                "bool": "Bool"}


def cpp_string(s: str) -> str:
    return 'R"dc_src(' + s + ')dc_src"'


def registry_cpp(records: list[dict], sources: list[str]) -> str:
    out = ["// <auto-generated/> by `python -m dotcompute_amd.generator` from " + ", ".join(sources) + ".",
           "// The kernel registry (what KernelRegistrationEmitter.GenerateKernelRegistry emits for C#,",
           "// src/Runtime/DotCompute.Generators/Kernel/Generation/KernelRegistrationEmitter.cs:40-113), with a",
           "// HIP slot per kernel: the entry point in dc_kernels_gfx950.hsaco and its generated source.",
           '#include "DotCompute/Runtime.hpp"', "", "namespace DotCompute {", "",
           "std::vector<KernelRegistrationInfo> Generated::KernelRegistry::GetAllKernels() {",
           "  std::vector<KernelRegistrationInfo> all;"]
    for r in records:
        km = r["km"]
        if not km.params and km.error:
            out.append(f"  // [Kernel] {km.full_name} is not registered: {km.error}")
            continue
        out.append("  {")
        out.append("    KernelRegistrationInfo k;")
        out.append(f'    k.Name = "{km.name}";')
        out.append(f'    k.FullName = "{km.full_name}";')
        out.append(f'    k.Namespace = "{km.namespace}";')
        out.append(f'    k.ContainingType = "{km.containing_type}";')
        out.append("    k.SupportedBackends = {" + ", ".join(f'"{b}"' for b in km.backends) + "};")
        out.append(f"    k.VectorSize = {km.vector_size};")
        out.append(f"    k.IsParallel = {'true' if km.is_parallel else 'false'};")
        out.append(f"    k.Dimensions = {r['dims']};")
        out.append("    k.Parameters = {")
        for p in km.params:
            et = ELEMENT_TYPE[p.element]
            read = p.name in r["reads"] or r["error"] is not None
            written = p.is_buffer and (p.name in r["writes"] or (r["error"] is not None and not p.read_only))
            covered = p.name in r["covered"] and not read
            out.append(f'        {{"{p.name}", ElementType::{et}, {str(p.is_buffer).lower()}, '
                       f'{str(p.read_only).lower()}, {str(read).lower()}, {str(written).lower()}, '
                       f'{str(covered).lower()}}},')
        out.append("    };")
        if r["entry"]:
            out.append(f'    k.HipEntryPoint = "{r["entry"]}";')
            out.append(f"    k.HipNeedsLength = {'true' if r['needs_length'] else 'false'};")
            out.append("    k.HipAbi = HipKernelAbi::Generated;")
            out.append(f"    k.HipSource = {cpp_string(r['source'])};")
        else:
            msg = r["error"].replace("\\", "\\\\").replace('"', '\\"')
            out.append(f'    k.HipDiagnostic = "{msg}";')
        out.append("    all.push_back(std::move(k));")
        out.append("  }")
    out += ["  return all;", "}", "", "}  // namespace DotCompute", ""]
    return "\n".join(out)


def kernels_hip(records: list[dict], sources: list[str]) -> str:
    out = ["// <auto-generated/> by `python -m dotcompute_amd.generator` from " + ", ".join(sources) + ".",
           "// gfx950 kernels translated from [Kernel] C# bodies; built into dc_kernels_gfx950.hsaco.",
           '#include "dc_gen_support.hpp"', ""]
    for r in records:
        if r["source"]:
            out.append(r["source"])
            out.append("")
        else:
            out.append(f"// [Kernel] {r['km'].full_name}: no HIP translation ({r['error']})")
            out.append("")
    return "\n".join(out)
