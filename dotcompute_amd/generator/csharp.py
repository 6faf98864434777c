"""Lexer, parser and type checker for the [Kernel] subset of C# that the HIP generator translates.

The subset is the one the reference's CUDA emitter handles (KernelExecutionMetadataEmitter.cs:
255-390: local declarations, expression statements, blocks, `if`/`else`, `return;`, binary,
assignment, unary, literal, identifier, element access, cast, KernelContext intrinsics and a
buffer's `.Length`), widened by `for`/`while`/`break`/`continue`, the conditional operator, `var`
and the Math/MathF calls Sqrt, Abs, Min and Max. Anything else raises Unsupported, and the kernel
is registered without a HIP entry point (the reference does the same for CUDA: GenerateCuda
returns null, :98-103).

Every expression gets its C# type (binary numeric promotion, C# spec 12.4.7), so the emitter can
write the conversions C# performs implicitly and C++ would perform differently (uint + int is
long in C#, unsigned int in C++; integer literals take the first of int, uint, long, ulong that
holds them).
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field


class Unsupported(Exception):
    """The construct is outside the translatable subset."""


# ---------------------------------------------------------------------------------------------
# Types
# ---------------------------------------------------------------------------------------------
INTEGRAL = ("sbyte", "byte", "short", "ushort", "int", "uint", "long", "ulong", "char")
FLOATING = ("float", "double")
NUMERIC = INTEGRAL + FLOATING
BITS = {"sbyte": 8, "byte": 8, "short": 16, "ushort": 16, "char": 16, "int": 32, "uint": 32, "long": 64,
        "ulong": 64, "float": 32, "double": 64}
SIGNED = {"sbyte", "short", "int", "long"}
BCL_NAMES = {"System.Single": "float", "System.Double": "double", "System.Int32": "int", "System.UInt32": "uint",
             "System.Int64": "long", "System.UInt64": "ulong", "System.Int16": "short", "System.UInt16": "ushort",
             "System.Byte": "byte", "System.SByte": "sbyte", "System.Boolean": "bool", "Single": "float",
             "Double": "double", "Int32": "int", "UInt32": "uint", "Int64": "long", "UInt64": "ulong",
             "Int16": "short", "UInt16": "ushort", "Byte": "byte", "SByte": "sbyte", "Boolean": "bool"}
KEYWORD_TYPES = {"bool", "float", "double", "int", "uint", "long", "ulong", "short", "ushort", "byte", "sbyte"}


def normalize_type(t: str) -> str:
    t = t.strip()
    return BCL_NAMES.get(t, t)


def promote_unary(t: str) -> str:
    """Unary numeric promotion: the small integral types become int."""
    if t in ("sbyte", "byte", "short", "ushort", "char"):
        return "int"
    return t


def promote_binary(a: str, b: str) -> str:
    """Binary numeric promotion (C# spec 12.4.7.3); decimal is not in the subset."""
    if a not in NUMERIC or b not in NUMERIC:
        raise Unsupported(f"arithmetic on {a} and {b}")
    if "double" in (a, b):
        return "double"
    if "float" in (a, b):
        return "float"
    if "ulong" in (a, b):
        other = b if a == "ulong" else a
        if other in SIGNED:
            raise Unsupported("ulong with a signed operand (a C# binding-time error)")
        return "ulong"
    if "long" in (a, b):
        return "long"
    if "uint" in (a, b):
        other = b if a == "uint" else a
        return "long" if other in ("sbyte", "short", "int") else "uint"
    return "int"


def int_constant(e) -> int | None:
    """Value of an int-typed constant expression (a literal, possibly negated), else None."""
    if isinstance(e, Lit) and e.ty == "int":
        return int(literal_type(e.text)[1])
    if isinstance(e, Unary) and e.op == "-" and e.ty == "int":
        v = int_constant(e.expr)
        return -v if v is not None else None
    return None


def promote_operands(a, b) -> str:
    """Binary numeric promotion with the constant conversions overload resolution applies: an int
    constant that fits converts implicitly to uint or ulong (C# 10.2.11), so `u + 1` is uint
    where `u + i` is long."""
    for x, y in ((a, b), (b, a)):
        if x.ty in ("uint", "ulong") and y.ty == "int":
            v = int_constant(y)
            if v is not None and 0 <= v <= (2**32 - 1 if x.ty == "uint" else 2**64 - 1):
                return x.ty
    return promote_binary(a.ty, b.ty)


def literal_type(text: str) -> tuple[str, str]:
    """C# type of a numeric literal and its digits/value text without suffix or separators."""
    t = text.replace("_", "")
    low = t.lower()
    if low.startswith("0x") or low.startswith("0b"):
        m = re.fullmatch(r"(0[xX][0-9a-fA-F]+|0[bB][01]+)([uUlL]*)", t)
        if not m:
            raise Unsupported(f"literal {text}")
        digits, suffix = m.group(1), m.group(2).lower()
        value = int(digits, 0)
        return _int_literal_type(value, suffix, text), str(value)
    m = re.fullmatch(r"([0-9]*\.?[0-9]*(?:[eE][+-]?[0-9]+)?)([fFdDmMuUlL]*)", t)
    if not m or not m.group(1) or m.group(1) == ".":
        raise Unsupported(f"literal {text}")
    digits, suffix = m.group(1), m.group(2).lower()
    if suffix == "m":
        raise Unsupported("decimal literals")
    is_real = "." in digits or "e" in digits.lower() or suffix in ("f", "d")
    if is_real:
        if suffix in ("u", "l", "ul", "lu"):
            raise Unsupported(f"literal {text}")
        return ("float" if suffix == "f" else "double"), digits
    return _int_literal_type(int(digits), suffix, text), digits


def _int_literal_type(value: int, suffix: str, text: str) -> str:
    if suffix == "":
        for t, hi in (("int", 2**31 - 1), ("uint", 2**32 - 1), ("long", 2**63 - 1), ("ulong", 2**64 - 1)):
            if value <= hi:
                return t
    elif suffix == "u":
        for t, hi in (("uint", 2**32 - 1), ("ulong", 2**64 - 1)):
            if value <= hi:
                return t
    elif suffix == "l":
        for t, hi in (("long", 2**63 - 1), ("ulong", 2**64 - 1)):
            if value <= hi:
                return t
    elif suffix in ("ul", "lu"):
        if value <= 2**64 - 1:
            return "ulong"
    raise Unsupported(f"literal {text}")


# ---------------------------------------------------------------------------------------------
# Lexer
# ---------------------------------------------------------------------------------------------
_TOKEN = re.compile(r"""
    (?P<ws>\s+|//[^\n]*|/\*.*?\*/)
  | (?P<num>(?:0[xX][0-9a-fA-F_]+|0[bB][01_]+)[uUlL]*|(?:[0-9][0-9_]*(?:\.[0-9][0-9_]*)?|\.[0-9][0-9_]*)(?:[eE][+-]?[0-9]+)?[fFdDmMuUlL]*)
  | (?P<str>"(?:\\.|[^"\\])*"|'(?:\\.|[^'\\])*')
  | (?P<id>@?[A-Za-z_][A-Za-z0-9_]*)
  | (?P<op><<=|>>>=|>>=|>>>|\?\?=|=>|&&|\|\||==|!=|<=|>=|<<|>>|\+\+|--|\+=|-=|\*=|/=|%=|&=|\|=|\^=|\?\?|\?\.|::|[{}()\[\];,.:?+\-*/%&|^!~<>=#])
""", re.VERBOSE | re.DOTALL)


@dataclass
class Tok:
    kind: str
    text: str
    line: int


def tokenize(src: str) -> list[Tok]:
    out, pos, line = [], 0, 1
    while pos < len(src):
        m = _TOKEN.match(src, pos)
        if not m:
            raise Unsupported(f"cannot tokenize near line {line}: {src[pos:pos + 20]!r}")
        kind = m.lastgroup
        text = m.group(kind)
        if kind != "ws":
            out.append(Tok(kind, text, line))
        line += text.count("\n")
        pos = m.end()
    out.append(Tok("eof", "", line))
    return out


# ---------------------------------------------------------------------------------------------
# AST
# ---------------------------------------------------------------------------------------------
@dataclass
class Expr:
    ty: str = field(default="", init=False)  # C# type after checking


@dataclass
class Lit(Expr):
    text: str


@dataclass
class BoolLit(Expr):
    value: bool


@dataclass
class Name(Expr):
    ident: str


@dataclass
class Intrinsic(Expr):
    kind: str  # ThreadId / BlockId / BlockDim / GridDim
    axis: str  # X / Y / Z


@dataclass
class Length(Expr):
    buffer: str


@dataclass
class Index(Expr):
    buffer: str
    index: Expr


@dataclass
class Call(Expr):
    func: str  # Math.Sqrt, MathF.Abs, ...
    args: list


@dataclass
class Cast(Expr):
    to: str
    expr: Expr


@dataclass
class Unary(Expr):
    op: str
    expr: Expr
    postfix: bool = False


@dataclass
class Binary(Expr):
    op: str
    left: Expr
    right: Expr
    operand_ty: str = ""  # promoted operand type (comparisons, arithmetic)


@dataclass
class Cond(Expr):
    cond: Expr
    a: Expr
    b: Expr


@dataclass
class Assign(Expr):
    op: str  # "=", "+=", ...
    target: Expr  # Name or Index
    value: Expr
    operand_ty: str = ""


@dataclass
class Stmt:
    pass


@dataclass
class Block(Stmt):
    body: list


@dataclass
class LocalDecl(Stmt):
    ty: str  # "var" is resolved by the checker
    names: list  # [(name, init Expr | None)]


@dataclass
class ExprStmt(Stmt):
    expr: Expr


@dataclass
class If(Stmt):
    cond: Expr
    then: Stmt
    other: Stmt | None


@dataclass
class Return(Stmt):
    pass


@dataclass
class For(Stmt):
    init: list  # LocalDecl or ExprStmt list
    cond: Expr | None
    iters: list  # Expr list
    body: Stmt


@dataclass
class While(Stmt):
    cond: Expr
    body: Stmt


@dataclass
class Break(Stmt):
    pass


@dataclass
class Continue(Stmt):
    pass


@dataclass
class Param:
    name: str
    type_text: str
    is_buffer: bool
    element: str  # buffer element type or scalar type (C# keyword)
    read_only: bool  # ReadOnlySpan<T>


@dataclass
class KernelMethod:
    name: str
    namespace: str
    containing_type: str
    backends: list
    vector_size: int
    is_parallel: bool
    params: list
    body_tokens: list
    body: Block | None = None
    error: str | None = None  # why no HIP translation exists
    line: int = 0

    @property
    def full_name(self) -> str:
        return f"{self.containing_type}.{self.name}" if self.containing_type else self.name


# ---------------------------------------------------------------------------------------------
# File-level scan: namespaces, types and [Kernel] methods
# ---------------------------------------------------------------------------------------------
BACKEND_FLAGS = {"CPU": 1, "CUDA": 2, "Metal": 4, "OpenCL": 8, "HIP": 16}


def find_kernels(src: str) -> list[KernelMethod]:
    toks = tokenize(src)
    kernels: list[KernelMethod] = []
    scope: list[tuple[str, str]] = []  # (kind, name) per open brace
    file_ns = ""
    pending: tuple[str, str] | None = None
    i = 0
    while toks[i].kind != "eof":
        t = toks[i]
        if t.text == "namespace":
            j = i + 1
            parts = []
            while toks[j].kind == "id" or toks[j].text == ".":
                parts.append(toks[j].text)
                j += 1
            if toks[j].text == ";":
                file_ns = "".join(parts)
                i = j + 1
                continue
            pending = ("ns", "".join(parts))
            i = j
            continue
        if t.text in ("class", "struct", "record", "interface") and toks[i + 1].kind == "id":
            pending = ("type", toks[i + 1].text)
            i += 2
            continue
        if t.text == "{":
            scope.append(pending or ("block", ""))
            pending = None
            i += 1
            continue
        if t.text == "}":
            if scope:
                scope.pop()
            i += 1
            continue
        if t.text == "[" and toks[i + 1].text == "Kernel" and toks[i + 2].text in ("]", "("):
            attr_end = _match(toks, i, "[", "]")
            backends, vector_size, is_parallel = _kernel_attribute(toks[i + 2:attr_end])
            j = attr_end + 1
            while toks[j].text == "[":  # other attributes
                j = _match(toks, j, "[", "]") + 1
            mods = set()
            while toks[j].text in ("public", "private", "internal", "protected", "static", "unsafe", "new"):
                mods.add(toks[j].text)
                j += 1
            if toks[j].text != "void" or toks[j + 1].kind != "id" or toks[j + 2].text != "(":
                raise Unsupported(f"line {toks[j].line}: a [Kernel] method must be `static void Name(...)`")
            name = toks[j + 1].text
            pend = _match(toks, j + 2, "(", ")")
            param_error = None
            try:
                params = _params(toks[j + 3:pend])
            except Unsupported as e:  # registered without parameters; the registry leaves it out
                params, param_error = [], str(e)
            if toks[pend + 1].text != "{":
                raise Unsupported(f"line {toks[pend + 1].line}: kernel {name} has no block body")
            bend = _match(toks, pend + 1, "{", "}")
            ns = ".".join([n for k, n in scope if k == "ns" and n] or ([file_ns] if file_ns else []))
            types = ".".join(n for k, n in scope if k == "type")
            containing = f"{ns}.{types}" if ns and types else (types or ns)
            km = KernelMethod(name, ns, containing, backends, vector_size, is_parallel, params,
                              toks[pend + 2:bend] + [Tok("eof", "", toks[bend].line)], line=toks[j].line)
            if param_error:
                km.error = param_error
            kernels.append(km)
            i = bend + 1
            continue
        i += 1
    return kernels


def _match(toks, i, open_, close):
    depth = 0
    for j in range(i, len(toks)):
        if toks[j].text == open_:
            depth += 1
        elif toks[j].text == close:
            depth -= 1
            if depth == 0:
                return j
    raise Unsupported(f"unbalanced {open_}{close} from line {toks[i].line}")


def _kernel_attribute(toks) -> tuple[list, int, bool]:
    backends, vector_size, is_parallel = 1, 8, True  # KernelAttribute.cs:32 and defaults
    if toks and toks[0].text == "(":
        args = toks[1:-1] if toks[-1].text == ")" else toks[1:]
        k = 0
        while k < len(args):
            if args[k].kind == "id" and k + 1 < len(args) and args[k + 1].text == "=":
                key = args[k].text
                e = k + 2
                val = []
                while e < len(args) and args[e].text != ",":
                    val.append(args[e])
                    e += 1
                if key == "Backends":
                    backends = 0
                    for v in val:
                        if v.kind == "id" and v.text in BACKEND_FLAGS:
                            backends |= BACKEND_FLAGS[v.text]
                        elif v.text == "All":
                            backends |= 1 | 2 | 4 | 8
                elif key == "VectorSize" and val:
                    vector_size = int(val[0].text)
                elif key == "IsParallel" and val:
                    is_parallel = val[0].text == "true"
                k = e + 1
            else:
                k += 1
    names = [n for n, f in BACKEND_FLAGS.items() if backends & f]
    return names, vector_size, is_parallel


def _params(toks) -> list[Param]:
    params = []
    cur: list[Tok] = []
    depth = 0
    for t in toks + [Tok("op", ",", 0)]:
        if t.text == "<":
            depth += 1
        elif t.text == ">":
            depth -= 1
        if t.text == "," and depth == 0:
            if cur:
                params.append(_param(cur))
            cur = []
        else:
            cur.append(t)
    return params


def _param(toks) -> Param:
    if toks[0].text in ("ref", "out", "in", "params", "this"):
        raise Unsupported(f"parameter modifier `{toks[0].text}`")
    name = toks[-1].text
    type_text = "".join(t.text for t in toks[:-1])
    m = re.fullmatch(r"(ReadOnlySpan|Span)<(.+)>", type_text)
    if m:
        elem = normalize_type(m.group(2))
        if elem not in NUMERIC or elem == "char":
            raise Unsupported(f"buffer element type {elem}")
        return Param(name, type_text, True, elem, m.group(1) == "ReadOnlySpan")
    if type_text.endswith("[]"):
        elem = normalize_type(type_text[:-2])
        if elem not in NUMERIC or elem == "char":
            raise Unsupported(f"buffer element type {elem}")
        return Param(name, type_text, True, elem, False)
    t = normalize_type(type_text)
    if t not in KEYWORD_TYPES:
        raise Unsupported(f"parameter type {type_text}")
    return Param(name, type_text, False, t, False)


# ---------------------------------------------------------------------------------------------
# Statement / expression parser
# ---------------------------------------------------------------------------------------------
class Parser:
    def __init__(self, toks: list[Tok]):
        self.t = toks
        self.i = 0

    def peek(self, k=0) -> Tok:
        return self.t[self.i + k]

    def next(self) -> Tok:
        tok = self.t[self.i]
        self.i += 1
        return tok

    def expect(self, text: str) -> Tok:
        tok = self.next()
        if tok.text != text:
            raise Unsupported(f"line {tok.line}: expected `{text}`, found `{tok.text}`")
        return tok

    def block_body(self) -> Block:
        body = []
        while self.peek().kind != "eof":
            body.append(self.statement())
        return Block(body)

    def statement(self) -> Stmt:
        t = self.peek()
        if t.text == "{":
            self.next()
            body = []
            while self.peek().text != "}":
                if self.peek().kind == "eof":
                    raise Unsupported("unterminated block")
                body.append(self.statement())
            self.next()
            return Block(body)
        if t.text == ";":
            self.next()
            return Block([])
        if t.text == "if":
            self.next()
            self.expect("(")
            c = self.expression()
            self.expect(")")
            then = self.statement()
            other = None
            if self.peek().text == "else":
                self.next()
                other = self.statement()
            return If(c, then, other)
        if t.text == "return":
            self.next()
            if self.peek().text != ";":
                raise Unsupported(f"line {t.line}: `return` with a value")
            self.next()
            return Return()
        if t.text == "break":
            self.next()
            self.expect(";")
            return Break()
        if t.text == "continue":
            self.next()
            self.expect(";")
            return Continue()
        if t.text == "while":
            self.next()
            self.expect("(")
            c = self.expression()
            self.expect(")")
            return While(c, self.statement())
        if t.text == "for":
            self.next()
            self.expect("(")
            init = []
            if self.peek().text != ";":
                if self.is_decl_start():
                    init.append(self.local_decl())
                else:
                    init.append(ExprStmt(self.expression()))
                    while self.peek().text == ",":
                        self.next()
                        init.append(ExprStmt(self.expression()))
            self.expect(";")
            cond = None if self.peek().text == ";" else self.expression()
            self.expect(";")
            iters = []
            if self.peek().text != ")":
                iters.append(self.expression())
                while self.peek().text == ",":
                    self.next()
                    iters.append(self.expression())
            self.expect(")")
            return For(init, cond, iters, self.statement())
        if t.text in ("do", "switch", "foreach", "goto", "try", "throw", "lock", "using", "unsafe", "fixed",
                      "checked", "unchecked", "yield", "const", "stackalloc"):
            raise Unsupported(f"line {t.line}: `{t.text}` statements")
        if self.is_decl_start():
            d = self.local_decl()
            self.expect(";")
            return d
        e = self.expression()
        self.expect(";")
        if not isinstance(e, (Assign, Unary)) or (isinstance(e, Unary) and e.op not in ("++", "--")):
            raise Unsupported(f"line {t.line}: expression statement without an effect")
        return ExprStmt(e)

    def is_decl_start(self) -> bool:
        t = self.peek()
        if t.kind != "id":
            return False
        if t.text == "System" and self.peek(1).text == ".":
            return self.peek(3).kind == "id"
        # `Type name` followed by `=`, `;` or `,`: a declaration (the checker rejects types outside
        # the subset, e.g. `string s = ...`)
        return self.peek(1).kind == "id" and self.peek(2).text in ("=", ";", ",")

    def local_decl(self) -> LocalDecl:
        ty = self.next().text
        if ty == "System":
            self.expect(".")
            ty = "System." + self.next().text
        ty = normalize_type(ty)
        names = []
        while True:
            name = self.next()
            if name.kind != "id":
                raise Unsupported(f"line {name.line}: bad declaration")
            init = None
            if self.peek().text == "=":
                self.next()
                init = self.expression()
            names.append((name.text, init))
            if self.peek().text != ",":
                break
            self.next()
        return LocalDecl(ty, names)

    # precedence climbing, C# precedence table
    def expression(self) -> Expr:
        return self.assignment()

    ASSIGN_OPS = ("=", "+=", "-=", "*=", "/=", "%=", "&=", "|=", "^=", "<<=", ">>=")

    def assignment(self) -> Expr:
        left = self.conditional()
        if self.peek().text in self.ASSIGN_OPS:
            op = self.next().text
            if not isinstance(left, (Name, Index)):
                raise Unsupported("assignment to something other than a local or a buffer element")
            return Assign(op, left, self.assignment())
        if self.peek().text in ("??=", ">>>="):
            raise Unsupported(f"operator {self.peek().text}")
        return left

    def conditional(self) -> Expr:
        c = self.binary(0)
        if self.peek().text == "?":
            self.next()
            a = self.assignment()
            self.expect(":")
            b = self.assignment()
            return Cond(c, a, b)
        return c

    LEVELS = [("||",), ("&&",), ("|",), ("^",), ("&",), ("==", "!="), ("<", ">", "<=", ">="), ("<<", ">>"),
              ("+", "-"), ("*", "/", "%")]

    def binary(self, level: int) -> Expr:
        if level == len(self.LEVELS):
            return self.unary()
        left = self.binary(level + 1)
        while self.peek().text in self.LEVELS[level]:
            op = self.next().text
            right = self.binary(level + 1)
            left = Binary(op, left, right)
        if self.peek().text in ("??", ">>>", "is", "as"):
            raise Unsupported(f"operator {self.peek().text}")
        return left

    def unary(self) -> Expr:
        t = self.peek()
        if t.text in ("+", "-", "!", "~"):
            self.next()
            return Unary(t.text, self.unary())
        if t.text in ("++", "--"):
            self.next()
            return Unary(t.text, self.unary())
        if t.text == "(" and self.peek(1).text in KEYWORD_TYPES and self.peek(2).text == ")":
            self.next()
            ty = normalize_type(self.next().text)
            self.next()
            return Cast(ty, self.unary())
        return self.postfix(self.primary())

    def postfix(self, e: Expr) -> Expr:
        while True:
            t = self.peek()
            if t.text == "[":
                self.next()
                idx = self.expression()
                if self.peek().text == ",":
                    raise Unsupported("multi-dimensional indexing")
                self.expect("]")
                if not isinstance(e, Name):
                    raise Unsupported("indexing something other than a buffer parameter")
                e = Index(e.ident, idx)
            elif t.text in ("++", "--"):
                self.next()
                e = Unary(t.text, e, postfix=True)
            else:
                return e

    def primary(self) -> Expr:
        t = self.next()
        if t.kind == "num":
            return Lit(t.text)
        if t.kind == "str":
            raise Unsupported("string and char literals")
        if t.text == "(":
            e = self.expression()
            self.expect(")")
            return e
        if t.text in ("true", "false"):
            return BoolLit(t.text == "true")
        if t.kind == "id":
            parts = [t.text]
            while self.peek().text == "." and self.peek(1).kind == "id":
                self.next()
                parts.append(self.next().text)
            if self.peek().text == "(":
                self.next()
                args = []
                if self.peek().text != ")":
                    args.append(self.expression())
                    while self.peek().text == ",":
                        self.next()
                        args.append(self.expression())
                self.expect(")")
                func = ".".join(parts)
                if func.startswith("System."):
                    func = func[len("System."):]
                return Call(func, args)
            return self.member_chain(parts, t.line)
        raise Unsupported(f"line {t.line}: unexpected `{t.text}`")

    def member_chain(self, parts: list, line: int) -> Expr:
        if len(parts) == 1:
            return Name(parts[0])
        # <root>.{ThreadId|BlockId|BlockDim|GridDim}.{X|Y|Z}; the root is not checked, as in the
        # reference's TryClassifyIntrinsic (KernelExecutionMetadataEmitter.cs:415-452).
        if len(parts) >= 2 and parts[-1] in ("X", "Y", "Z") and parts[-2] in ("ThreadId", "BlockId", "BlockDim",
                                                                                "GridDim"):
            return Intrinsic(parts[-2], parts[-1])
        if len(parts) == 2 and parts[1] == "Length":
            return Length(parts[0])
        raise Unsupported(f"line {line}: member access {'.'.join(parts)}")


# ---------------------------------------------------------------------------------------------
# Type checker
# ---------------------------------------------------------------------------------------------
MATH_FUNCS = {"Math.Sqrt", "MathF.Sqrt", "Math.Abs", "MathF.Abs", "Math.Min", "MathF.Min", "Math.Max", "MathF.Max"}


class Checker:
    def __init__(self, params: list[Param]):
        self.buffers = {p.name: p for p in params if p.is_buffer}
        self.scopes: list[dict] = [{p.name: p.element for p in params if not p.is_buffer}]
        self.uses_length = False
        self.dims = 1
        self.reads: set[str] = set()
        self.writes: set[str] = set()
        self.loop_depth = 0

    def lookup(self, name: str) -> str:
        for s in reversed(self.scopes):
            if name in s:
                return s[name]
        if name in self.buffers:
            raise Unsupported(f"buffer `{name}` used as a value")
        raise Unsupported(f"unknown identifier `{name}`")

    def stmt(self, s: Stmt) -> None:
        if isinstance(s, Block):
            self.scopes.append({})
            for x in s.body:
                self.stmt(x)
            self.scopes.pop()
        elif isinstance(s, LocalDecl):
            for i, (name, init) in enumerate(s.names):
                if init is not None:
                    self.expr(init)
                if s.ty == "var":
                    if init is None:
                        raise Unsupported("`var` without an initialiser")
                    ty = init.ty
                    if ty == "null":
                        raise Unsupported("`var` of null")
                else:
                    ty = s.ty
                    if ty not in KEYWORD_TYPES:
                        raise Unsupported(f"local of type {ty}")
                    if init is not None:
                        self.check_assignable(init, ty)
                if any(name in sc for sc in self.scopes) or name in self.buffers:
                    raise Unsupported(f"`{name}` shadows another variable")
                self.scopes[-1][name] = ty
            if s.ty == "var":
                s.ty = s.names and self.scopes[-1][s.names[0][0]]
                if len({self.scopes[-1][n] for n, _ in s.names}) > 1:
                    raise Unsupported("`var` declaring variables of different types")
        elif isinstance(s, ExprStmt):
            self.expr(s.expr, statement=True)
        elif isinstance(s, If):
            self.expr(s.cond)
            if s.cond.ty != "bool":
                raise Unsupported("if condition is not bool")
            self.stmt(s.then)
            if s.other is not None:
                self.stmt(s.other)
        elif isinstance(s, (Return,)):
            pass
        elif isinstance(s, (Break, Continue)):
            if self.loop_depth == 0:
                raise Unsupported("break/continue outside a loop")
        elif isinstance(s, For):
            self.scopes.append({})
            for x in s.init:
                self.stmt(x) if isinstance(x, LocalDecl) else self.expr(x.expr, statement=True)
            if s.cond is not None:
                self.expr(s.cond)
                if s.cond.ty != "bool":
                    raise Unsupported("for condition is not bool")
            for x in s.iters:
                self.expr(x, statement=True)
            self.loop_depth += 1
            self.stmt(s.body)
            self.loop_depth -= 1
            self.scopes.pop()
        elif isinstance(s, While):
            self.expr(s.cond)
            if s.cond.ty != "bool":
                raise Unsupported("while condition is not bool")
            self.loop_depth += 1
            self.stmt(s.body)
            self.loop_depth -= 1
        else:
            raise Unsupported(f"statement {type(s).__name__}")

    def check_assignable(self, e: Expr, to: str) -> None:
        """C# implicit conversions the subset allows (identity, numeric widening, int constants)."""
        if e.ty == to:
            return
        if to == "bool" or e.ty == "bool":
            raise Unsupported(f"no implicit conversion from {e.ty} to {to}")
        if isinstance(e, Lit) and e.ty == "int" and to in INTEGRAL:
            return  # constant expression conversion (C# 10.2.11); the emitter casts
        widen = {
            "sbyte": {"short", "int", "long", "float", "double"},
            "byte": {"short", "ushort", "int", "uint", "long", "ulong", "float", "double"},
            "short": {"int", "long", "float", "double"},
            "ushort": {"int", "uint", "long", "ulong", "float", "double"},
            "int": {"long", "float", "double"},
            "uint": {"long", "ulong", "float", "double"},
            "long": {"float", "double"},
            "ulong": {"float", "double"},
            "float": {"double"},
        }
        if to not in widen.get(e.ty, set()):
            raise Unsupported(f"no implicit conversion from {e.ty} to {to}")

    def expr(self, e: Expr, statement: bool = False) -> str:
        ty = self._expr(e, statement)
        e.ty = ty
        return ty

    def _expr(self, e: Expr, statement: bool) -> str:
        if isinstance(e, Lit):
            return literal_type(e.text)[0]
        if isinstance(e, BoolLit):
            return "bool"
        if isinstance(e, Name):
            return self.lookup(e.ident)
        if isinstance(e, Intrinsic):
            if e.axis == "Z":
                self.dims = 3
            elif e.axis == "Y":
                self.dims = max(self.dims, 2)
            return "int"
        if isinstance(e, Length):
            if e.buffer not in self.buffers:
                raise Unsupported(f"`.Length` of `{e.buffer}`, which is not a buffer parameter")
            self.uses_length = True
            return "int"
        if isinstance(e, Index):
            if e.buffer not in self.buffers:
                raise Unsupported(f"indexing `{e.buffer}`, which is not a buffer parameter")
            it = self.expr(e.index)
            if it not in ("int", "short", "ushort", "byte", "sbyte", "char"):
                raise Unsupported(f"span index of type {it} (the indexer takes int)")
            self.reads.add(e.buffer)
            return self.buffers[e.buffer].element
        if isinstance(e, Cast):
            t = self.expr(e.expr)
            if (t == "bool") != (e.to == "bool"):
                raise Unsupported(f"cast between bool and {e.to if t == 'bool' else t}")
            return e.to
        if isinstance(e, Call):
            if e.func not in MATH_FUNCS:
                raise Unsupported(f"call to {e.func}")
            tys = [self.expr(a) for a in e.args]
            fname = e.func.split(".")[1]
            want = 1 if fname in ("Sqrt", "Abs") else 2
            if len(tys) != want:
                raise Unsupported(f"{e.func} with {len(tys)} arguments")
            if e.func.startswith("MathF."):
                for a in e.args:
                    if a.ty not in ("float",):
                        self.check_assignable(a, "float")
                return "float"
            if fname == "Sqrt":
                return "double"
            if fname == "Abs":
                return promote_unary(tys[0]) if tys[0] not in ("byte", "ushort") else "int"
            return promote_operands(e.args[0], e.args[1])
        if isinstance(e, Unary):
            t = self.expr(e.expr)
            if e.op in ("++", "--"):
                if not isinstance(e.expr, (Name, Index)):
                    raise Unsupported("++/-- of something other than a variable or element")
                if isinstance(e.expr, Index):
                    if not statement:
                        raise Unsupported("++/-- of a buffer element inside an expression")
                    self.writes.add(e.expr.buffer)
                if t not in NUMERIC:
                    raise Unsupported(f"++/-- on {t}")
                return t
            if e.op == "!":
                if t != "bool":
                    raise Unsupported("! on a non-bool")
                return "bool"
            if e.op == "~":
                p = promote_unary(t)
                if p not in ("int", "uint", "long", "ulong"):
                    raise Unsupported(f"~ on {t}")
                return p
            if t not in NUMERIC:
                raise Unsupported(f"unary {e.op} on {t}")
            p = promote_unary(t)
            if e.op == "-":
                if p == "uint":
                    return "long"
                if p == "ulong":
                    raise Unsupported("unary minus on ulong")
            return p
        if isinstance(e, Binary):
            a, b = self.expr(e.left), self.expr(e.right)
            op = e.op
            if op in ("&&", "||"):
                if a != "bool" or b != "bool":
                    raise Unsupported(f"{op} on non-bool operands")
                return "bool"
            if op in ("&", "|", "^") and a == "bool" and b == "bool":
                e.operand_ty = "bool"
                return "bool"
            if op in ("==", "!=") and a == "bool" and b == "bool":
                e.operand_ty = "bool"
                return "bool"
            if op in ("<<", ">>"):
                p = promote_unary(a)
                if p not in ("int", "uint", "long", "ulong"):
                    raise Unsupported(f"shift of {a}")
                if promote_unary(b) != "int":
                    raise Unsupported("shift count that is not int")
                e.operand_ty = p
                return p
            p = promote_operands(e.left, e.right)
            if op in ("&", "|", "^", "%") and p in FLOATING and op != "%":
                raise Unsupported(f"{op} on floating operands")
            e.operand_ty = p
            if op in ("==", "!=", "<", ">", "<=", ">="):
                return "bool"
            return p
        if isinstance(e, Cond):
            c = self.expr(e.cond)
            if c != "bool":
                raise Unsupported("?: condition is not bool")
            a, b = self.expr(e.a), self.expr(e.b)
            if a == b:
                return a
            if "bool" in (a, b):
                raise Unsupported("?: mixing bool and a number")
            return promote_operands(e.a, e.b)
        if isinstance(e, Assign):
            if not statement and e.op != "=":
                raise Unsupported("compound assignment inside an expression")
            if isinstance(e.target, Index):
                if not statement:
                    raise Unsupported("buffer element assignment inside an expression")
                if e.target.buffer not in self.buffers:
                    raise Unsupported(f"`{e.target.buffer}` is not a buffer parameter")
                if self.buffers[e.target.buffer].read_only:
                    raise Unsupported(f"`{e.target.buffer}` is a ReadOnlySpan")
                it = self.expr(e.target.index)
                if it not in ("int", "short", "ushort", "byte", "sbyte", "char"):
                    raise Unsupported(f"span index of type {it}")
                tt = self.buffers[e.target.buffer].element
                self.writes.add(e.target.buffer)
                if e.op != "=":
                    self.reads.add(e.target.buffer)
            else:
                tt = self.lookup(e.target.ident)
                e.target.ty = tt
            vt = self.expr(e.value)
            if e.op == "=":
                self.check_assignable(e.value, tt)
            else:
                bop = e.op[:-1]
                if bop in ("<<", ">>"):
                    e.operand_ty = promote_unary(tt)
                    if e.operand_ty not in ("int", "uint", "long", "ulong") or promote_unary(vt) != "int":
                        raise Unsupported(f"shift of {tt} by {vt}")
                elif tt == "bool" and bop in ("&", "|", "^"):
                    if vt != "bool":
                        raise Unsupported(f"{e.op} of bool with {vt}")
                    e.operand_ty = "bool"
                else:
                    target = Name("__target")
                    target.ty = tt
                    e.operand_ty = promote_operands(target, e.value)
                    # x op= y is x = (T)(x op y), allowed when y converts implicitly to T (C# 12.21.4)
                    self.check_assignable(e.value, tt)
            return tt
        raise Unsupported(f"expression {type(e).__name__}")


def analyse(kernel: KernelMethod) -> Checker:
    """Parses and type-checks the kernel body (raises Unsupported)."""
    p = Parser(kernel.body_tokens)
    kernel.body = p.block_body()
    c = Checker(kernel.params)
    if len([q for q in kernel.params if q.is_buffer]) > 16:
        raise Unsupported("more than 16 buffer parameters")
    c.stmt(kernel.body)
    return c
