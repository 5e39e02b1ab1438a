"""A small Lua 5.1 interpreter with a LuaJIT-style ``ffi`` over ctypes, written
for the tests: it runs lanternl_amd/lua/luatl_adapter.lua and
lanternl_amd/lua/lanternl_lm.lua themselves (against the real library on the
GPU) where no Lua runtime exists (none in this image or on the GPU box).

It covers the language those modules and their tests use: locals, closures
(each capturing the variables it names), numeric and generic ``for``,
``while``, ``repeat``, multiple results, varargs, tables with metatables
(``__index``, ``__newindex``, ``__call``), method calls, ``pcall``/``error``
with Lua's position prefixes, and the parts of ``string``, ``table``,
``math``, ``os`` and ``debug`` those files call.  ``ffi`` supports ``cdef`` of
C prototypes and plain structs (a second declaration of a name raises, as in
LuaJIT), ``load``, ``new``, ``typeof``, ``cast``, ``gc``, ``string``, pointer
and array indexing, pointer arithmetic, NULL comparisons, Lua strings passed
as ``const char*``, and 64-bit integers from C boxed as LuaJIT boxes them.
Anything outside that raises, so a test cannot pass on an unimplemented
feature.  Test infrastructure only; it is not part of the product.
"""
import ctypes
import math
import os
import re
import weakref

from tests.lua_lint import BINPRI, UNARY_PRI, LuaSyntaxError, tokenize


# ---------------------------------------------------------------- values
class LuaError(Exception):
    """A Lua error; `value` is what error() was given (any Lua value)."""

    def __init__(self, value):
        super().__init__(value)
        self.value = value


class LuaTable:
    __slots__ = ("d", "meta", "__weakref__")

    def __init__(self, d=None):
        self.d = {} if d is None else d
        self.meta = None

    @staticmethod
    def key(k):
        if isinstance(k, float) and k.is_integer():
            return int(k)
        if isinstance(k, float) and math.isnan(k):
            raise LuaError("table index is NaN")
        if isinstance(k, CInt64):
            raise LuaError("a 64-bit integer cdata used as a table key (LuaJIT keys cdata by identity); "
                           "convert it with tonumber()")
        if isinstance(k, bool):
            return k
        return k

    def rawget(self, k):
        if isinstance(k, float) and math.isnan(k):
            return None                 # reading t[NaN] is nil; only assignment raises
        return self.d.get(self.key(k))

    def rawset(self, k, v):
        k = self.key(k)
        if k is None:
            raise LuaError("table index is nil")
        if v is None:
            self.d.pop(k, None)
        else:
            self.d[k] = v

    def length(self):
        n = 0
        d = self.d
        while (n + 1) in d:
            n += 1
        return n

    @classmethod
    def from_list(cls, seq):
        return cls({i + 1: v for i, v in enumerate(seq)})

    def to_list(self):
        return [self.d[i] for i in range(1, self.length() + 1)]


class CInt64:
    """A 64-bit integer cdata.  LuaJIT boxes every int64_t / uint64_t value it
    reads from C (a return value, an array element, a struct field): tonumber()
    converts it, arithmetic with numbers stays 64-bit, comparisons work; here
    math functions, 'for' limits, concatenation and use as a table key refuse
    it, so a missing tonumber() in the Lua under test fails."""
    __slots__ = ("v", "unsigned")

    def __init__(self, v, unsigned=False):
        v = int(v) % (1 << 64)
        if not unsigned and v >= 1 << 63:
            v -= 1 << 64
        self.v, self.unsigned = v, unsigned


class LuaFunction:
    __slots__ = ("params", "vararg", "body", "scopes", "name", "vm", "src", "chunk")

    def __init__(self, params, vararg, body, scopes, name, vm, chunk="?"):
        self.params, self.vararg, self.body, self.scopes, self.name, self.vm = params, vararg, body, scopes, name, vm
        self.chunk = chunk
        self.src = chunk[1:] if chunk.startswith("@") else f'[string "{chunk}"]'

    def __call__(self, *args):
        return self.vm.call_function(self, list(args))


class _Break(Exception):
    pass


class _Return(Exception):
    def __init__(self, values):
        super().__init__()
        self.values = values


# ---------------------------------------------------------------- parser -> AST
class _AstParser:
    def __init__(self, text, chunkname):
        self.t = tokenize(text)
        self.p = 0
        self.chunk = chunkname
        self.fstack = []       # names referenced inside each function being parsed
        self.vstack = [True]   # whether each enclosing function is vararg (the chunk is)

    def ref(self, nm):
        for s in self.fstack:
            s.add(nm)

    def peek(self, k=0):
        return self.t[self.p + k]

    def check(self, kind, value=None):
        tk = self.t[self.p]
        return tk[0] == kind and (value is None or tk[1] == value)

    def accept(self, kind, value=None):
        if self.check(kind, value):
            self.p += 1
            return True
        return False

    def expect(self, kind, value=None):
        tk = self.t[self.p]
        if not self.check(kind, value):
            raise LuaSyntaxError(f"{self.chunk}:{tk[2]}: expected {value or kind}, got {tk[1]!r}")
        self.p += 1
        return tk

    def name(self):
        return self.expect("name")[1]

    def block_follow(self):
        tk = self.peek()
        return tk[0] == "eof" or (tk[0] == "kw" and tk[1] in ("else", "elseif", "end", "until"))

    def block(self):
        stmts = []
        while not self.block_follow():
            line = self.peek()[2]
            if self.accept("kw", "return"):
                exprs = [] if self.block_follow() or self.check("op", ";") else self.explist()
                self.accept("op", ";")
                stmts.append(("return", exprs, line))
                break
            if self.accept("kw", "break"):
                stmts.append(("break", line))
                self.accept("op", ";")
                continue
            stmts.append(self.statement())
            self.accept("op", ";")
        return stmts

    def statement(self):
        tk = self.peek()
        line = tk[2]
        if tk[0] == "kw":
            kw = tk[1]
            if self.accept("kw", "do"):
                b = self.block()
                self.expect("kw", "end")
                return ("do", b, line)
            if self.accept("kw", "while"):
                c = self.expr()
                self.expect("kw", "do")
                b = self.block()
                self.expect("kw", "end")
                return ("while", c, b, line)
            if self.accept("kw", "repeat"):
                b = self.block()
                self.expect("kw", "until")
                return ("repeat", b, self.expr(), line)
            if self.accept("kw", "if"):
                arms = []
                c = self.expr()
                self.expect("kw", "then")
                arms.append((c, self.block()))
                els = None
                while True:
                    if self.accept("kw", "elseif"):
                        c = self.expr()
                        self.expect("kw", "then")
                        arms.append((c, self.block()))
                    elif self.accept("kw", "else"):
                        els = self.block()
                    else:
                        break
                self.expect("kw", "end")
                return ("if", arms, els, line)
            if self.accept("kw", "for"):
                first = self.name()
                if self.accept("op", "="):
                    a = self.expr()
                    self.expect("op", ",")
                    b = self.expr()
                    c = self.expr() if self.accept("op", ",") else None
                    self.expect("kw", "do")
                    body = self.block()
                    self.expect("kw", "end")
                    return ("fornum", first, a, b, c, body, line)
                names = [first]
                while self.accept("op", ","):
                    names.append(self.name())
                self.expect("kw", "in")
                exprs = self.explist()
                self.expect("kw", "do")
                body = self.block()
                self.expect("kw", "end")
                return ("forin", names, exprs, body, line)
            if self.accept("kw", "function"):
                nm = self.name()
                self.ref(nm)
                target = ("name", nm, line)
                full = nm
                method = False
                while self.check("op", ".") or self.check("op", ":"):
                    method = self.peek()[1] == ":"
                    self.p += 1
                    key = self.name()
                    full += ("." if not method else ":") + key
                    target = ("index", target, ("str", key), line)
                    if method:
                        break
                f = self.funcbody(method, full, line)
                return ("assign", [target], [f], line)
            if self.accept("kw", "local"):
                if self.accept("kw", "function"):
                    nm = self.name()
                    return ("localfunc", nm, self.funcbody(False, nm, line), line)
                names = [self.name()]
                while self.accept("op", ","):
                    names.append(self.name())
                exprs = self.explist() if self.accept("op", "=") else []
                return ("local", names, exprs, line)
            if kw == "goto":
                raise LuaSyntaxError(f"{self.chunk}:{line}: goto is not supported by this interpreter")
        e = self.suffixedexp()
        if self.check("op", "=") or self.check("op", ","):
            targets = [e]
            while self.accept("op", ","):
                targets.append(self.suffixedexp())
            for t in targets:
                if t[0] not in ("name", "index"):
                    raise LuaSyntaxError(f"{self.chunk}:{line}: cannot assign to this expression")
            self.expect("op", "=")
            return ("assign", targets, self.explist(), line)
        if e[0] not in ("call", "method"):
            raise LuaSyntaxError(f"{self.chunk}:{line}: syntax error near {self.peek()[1]!r}")
        return ("callstat", e, line)

    def funcbody(self, method, name, line):
        refs = set()
        self.fstack.append(refs)
        try:
            return self._funcbody(method, name, line, refs)
        finally:
            self.fstack.pop()

    def _funcbody(self, method, name, line, refs):
        self.expect("op", "(")
        params = ["self"] if method else []
        vararg = False
        if not self.check("op", ")"):
            while True:
                if self.accept("op", "..."):
                    vararg = True
                    break
                params.append(self.name())
                if not self.accept("op", ","):
                    break
        self.expect("op", ")")
        self.vstack.append(vararg)
        body = self.block()
        self.vstack.pop()
        self.expect("kw", "end")
        return ("func", params, vararg, body, name, line, frozenset(refs), self.chunk)

    def explist(self):
        out = [self.expr()]
        while self.accept("op", ","):
            out.append(self.expr())
        return out

    def primaryexp(self):
        tk = self.peek()
        if tk[0] == "name":
            self.p += 1
            self.ref(tk[1])
            return ("name", tk[1], tk[2])
        if self.accept("op", "("):
            e = self.expr()
            self.expect("op", ")")
            return ("paren", e, tk[2])
        raise LuaSyntaxError(f"{self.chunk}:{tk[2]}: unexpected symbol {tk[1]!r}")

    def suffixedexp(self):
        e = self.primaryexp()
        while True:
            line = self.peek()[2]
            if self.accept("op", "."):
                e = ("index", e, ("str", self.name()), line)
            elif self.accept("op", "["):
                k = self.expr()
                self.expect("op", "]")
                e = ("index", e, k, line)
            elif self.accept("op", ":"):
                nm = self.name()
                e = ("method", e, nm, self.callargs(), line)
            elif self.check("op", "(") or self.check("op", "{") or self.check("str"):
                e = ("call", e, self.callargs(), line)
            else:
                return e

    def callargs(self):
        tk = self.peek()
        if tk[0] == "str":
            self.p += 1
            return [("str", _str_value(tk))]
        if self.check("op", "{"):
            return [self.table()]
        self.expect("op", "(")
        args = [] if self.check("op", ")") else self.explist()
        self.expect("op", ")")
        return args

    def table(self):
        line = self.expect("op", "{")[2]
        items = []
        while not self.check("op", "}"):
            if self.accept("op", "["):
                k = self.expr()
                self.expect("op", "]")
                self.expect("op", "=")
                items.append(("key", k, self.expr()))
            elif self.check("name") and self.peek(1)[0] == "op" and self.peek(1)[1] == "=":
                k = self.name()
                self.p += 1
                items.append(("key", ("str", k), self.expr()))
            else:
                items.append(("pos", None, self.expr()))
            if not (self.accept("op", ",") or self.accept("op", ";")):
                break
        self.expect("op", "}")
        return ("table", items, line)

    def simpleexp(self):
        tk = self.peek()
        if tk[0] == "num":
            self.p += 1
            return ("num", _lua_number(tk[1]))
        if tk[0] == "str":
            self.p += 1
            return ("str", _str_value(tk))
        if tk[0] == "kw" and tk[1] in ("nil", "true", "false"):
            self.p += 1
            return (tk[1],)
        if self.accept("op", "..."):
            if not self.vstack[-1]:
                raise LuaSyntaxError(f"{self.chunk}:{tk[2]}: cannot use '...' outside a vararg function")
            self.ref("...")
            return ("vararg",)
        if self.check("op", "{"):
            return self.table()
        if self.accept("kw", "function"):
            return self.funcbody(False, "anonymous", tk[2])
        return self.suffixedexp()

    def expr(self, limit=0):
        tk = self.peek()
        if (tk[0] == "kw" and tk[1] == "not") or (tk[0] == "op" and tk[1] in ("-", "#")):
            self.p += 1
            e = ("un", tk[1], self.expr(UNARY_PRI), tk[2])
        else:
            e = self.simpleexp()
        while True:
            tk = self.peek()
            op = tk[1] if tk[0] in ("op", "kw") else None
            if op not in BINPRI or BINPRI[op][0] <= limit:
                return e
            self.p += 1
            rhs = self.expr(BINPRI[op][1])
            e = (op, e, rhs, tk[2]) if op in ("and", "or") else ("bin", op, e, rhs, tk[2])


def _str_value(tk):
    if tk[3]:
        return tk[1][1:] if tk[1].startswith("\n") else tk[1]
    return _unescape(tk[1])


def _lua_number(s):
    s2 = re.sub(r"(?:[uU]?[lL][lL]|i)$", "", s)
    if s2.lower().startswith("0x"):
        return float(int(s2, 16))
    return float(s2)


_ESC = {"n": "\n", "t": "\t", "r": "\r", "a": "\a", "b": "\b", "f": "\f", "v": "\v", "\\": "\\", '"': '"',
        "'": "'", "\n": "\n"}


def _unescape(s):
    out, i = [], 0
    while i < len(s):
        c = s[i]
        if c != "\\":
            out.append(c)
            i += 1
            continue
        n = s[i + 1]
        if n in _ESC:
            out.append(_ESC[n])
            i += 2
        elif n.isdigit():
            m = re.match(r"\d{1,3}", s[i + 1:])
            out.append(chr(int(m.group(0))))
            i += 1 + m.end()
        else:
            raise LuaSyntaxError(f"invalid escape \\{n}")
    return "".join(out)


# ---------------------------------------------------------------- helpers
def tostr(v):
    if v is None:
        return "nil"
    if v is True:
        return "true"
    if v is False:
        return "false"
    if isinstance(v, float):
        if v.is_integer() and abs(v) < 1e15:
            return str(int(v))
        if math.isnan(v):
            return "nan" if math.copysign(1, v) > 0 else "-nan"
        if math.isinf(v):
            return "inf" if v > 0 else "-inf"
        return "%.14g" % v
    if isinstance(v, int):
        return str(v)
    if isinstance(v, str):
        return v
    if isinstance(v, CData):
        return f"cdata<{v.ct.name}>: 0x{v.address():x}"
    if isinstance(v, CInt64):
        return f"{v.v}{'ULL' if v.unsigned else 'LL'}"
    return f"{type(v).__name__}: 0x{id(v):x}"


def truthy(v):
    return v is not None and v is not False


def tonum(v):
    if isinstance(v, bool):
        return None
    if isinstance(v, (int, float)):
        return float(v)
    if isinstance(v, str):
        try:
            s = v.strip()
            return float(int(s, 16)) if s.lower().startswith("0x") else float(s)
        except ValueError:
            return None
    if isinstance(v, CData):
        return v.tonumber()
    return None


def lua_type(v):
    if v is None:
        return "nil"
    if isinstance(v, bool):
        return "boolean"
    if isinstance(v, (int, float)):
        return "number"
    if isinstance(v, str):
        return "string"
    if isinstance(v, LuaTable):
        return "table"
    if isinstance(v, (CData, CType, CInt64)):
        return "cdata"
    if callable(v):
        return "function"
    return "userdata"


# ---------------------------------------------------------------- Lua patterns (the subset the files use)
_PCLASS = {"a": "A-Za-z", "d": "0-9", "l": "a-z", "s": r"\s", "u": "A-Z", "w": "A-Za-z0-9", "x": "0-9A-Fa-f",
           "p": re.escape("!\"#$%&'()*+,-./:;<=>?@[\\]^_`{|}~"), "c": r"\x00-\x1f"}


def lua_pattern_to_re(p):
    out, i = [], 0
    while i < len(p):
        c = p[i]
        if c == "%":
            n = p[i + 1]
            if n.lower() in _PCLASS:
                cls = _PCLASS[n.lower()]
                out.append(f"[{cls}]" if n.islower() else f"[^{cls}]")
            else:
                out.append(re.escape(n))
            i += 2
        elif c == "[":
            j = i + 1
            body = []
            if j < len(p) and p[j] == "^":
                body.append("^")
                j += 1
            first = True
            while j < len(p) and (p[j] != "]" or first):
                first = False
                if p[j] == "%":
                    n = p[j + 1]
                    body.append(_PCLASS[n.lower()] if n.lower() in _PCLASS else re.escape(n))
                    j += 2
                elif p[j] == "\\":
                    body.append("\\\\")
                    j += 1
                else:
                    body.append(p[j] if p[j] not in "[]" else "\\" + p[j])
                    j += 1
            out.append("[" + "".join(body) + "]")
            i = j + 1
        elif c == "-":
            out.append("*?")
            i += 1
        elif c in "^$" and (i == 0 or i == len(p) - 1):
            out.append(c if c == "^" else r"\Z")
            i += 1
        elif c in ".()*+?":
            out.append(c)
            i += 1
        else:
            out.append(re.escape(c))
            i += 1
    return "".join(out)


# ---------------------------------------------------------------- ffi over ctypes
_CBASE = {"void": None, "char": ctypes.c_char, "int": ctypes.c_int, "unsigned int": ctypes.c_uint,
          "int32_t": ctypes.c_int32, "uint32_t": ctypes.c_uint32, "int64_t": ctypes.c_int64,
          "uint64_t": ctypes.c_uint64, "long long": ctypes.c_longlong, "unsigned long long": ctypes.c_ulonglong,
          "size_t": ctypes.c_size_t, "float": ctypes.c_float, "double": ctypes.c_double,
          "unsigned char": ctypes.c_ubyte, "long": ctypes.c_long}
_FLOATS = (ctypes.c_float, ctypes.c_double)


class CType:
    """A C type.  ``base`` is a ctypes scalar or Structure class (None for
    void), ``ptr`` the pointer depth; ``vla`` (``T[?]``) or ``arrn`` (``T[n]``)
    make it an array whose elements are ``base`` at depth ``ptr``."""

    def __init__(self, base, ptr=0, name="", vla=False, arrn=None):
        self.base, self.ptr, self.name, self.vla, self.arrn = base, ptr, name, vla, arrn

    def is_array(self):
        return self.vla or self.arrn is not None

    def elem(self):
        """The element type of an array or the pointee of a pointer."""
        e = self.__dict__.get("_elem")
        if e is None:
            e = self._elem = self._make_elem()
        return e

    def _make_elem(self):
        if self.is_array():
            return CType(self.base, self.ptr, self.name.split("[")[0].strip())
        if self.ptr == 0:
            raise LuaError(f"cdata<{self.name}> is neither an array nor a pointer")
        return CType(self.base, self.ptr - 1, self.name[:-1].strip() if self.name.endswith("*") else self.name)

    def scalar_ctype(self):
        """The ctypes type of one value of this (non-array) type."""
        if self.ptr:
            return ctypes.c_void_p
        if self.base is None:
            raise LuaError("void has no values")
        return self.base

    def size(self):
        return ctypes.sizeof(self.scalar_ctype()) if (self.ptr or self.base is not None) else 1

    def __call__(self, *args):
        return _ffi_new(self, *args)


class CData:
    """A C value.  Owned values (``ffi.new``) keep their ctypes object in
    ``obj``; pointers are an address (``addr``) and a type, and keep nothing
    alive, as in LuaJIT."""

    def __init__(self, ct, obj=None, addr=None):
        self.ct, self.obj, self.addr = ct, obj, addr

    def address(self):
        if self.addr is not None:
            return self.addr
        return ctypes.addressof(self.obj)

    def is_pointer(self):
        return self.addr is not None

    def tonumber(self):
        if self.is_pointer():
            return float(self.addr)
        if self.obj is not None and hasattr(self.obj, "value"):
            return float(self.obj.value)
        raise LuaError(f"cannot convert cdata<{self.ct.name}> to a number")

    def _struct(self):
        b = self.ct.base
        if isinstance(b, type) and issubclass(b, ctypes.Structure):
            if self.obj is not None and not self.ct.is_array():
                return self.obj
            if self.is_pointer() and self.ct.ptr == 1:
                return b.from_address(self.addr)
        return None

    def index(self, k):
        if isinstance(k, str):
            st = self._struct()
            if st is None or k not in {f[0] for f in type(st)._fields_}:
                raise LuaError(f"cdata<{self.ct.name}> has no field '{k}'")
            return _from_c(getattr(st, k), dict(type(st)._fields_)[k])
        et = self.ct.elem()
        i = int(k)
        if not self.is_pointer():
            v = self.obj[i]              # bounds-checked, unlike LuaJIT: an overrun fails the test
        else:
            v = et.scalar_ctype().from_address(self.addr + i * et.size()).value
        if et.ptr:
            return CData(et, addr=v or 0)
        return _from_c(v, et.base)

    def setindex(self, k, v):
        if isinstance(k, str):
            st = self._struct()
            ftype = dict(type(st)._fields_).get(k) if st is not None else None
            if ftype is None:
                raise LuaError(f"cdata<{self.ct.name}> has no field '{k}'")
            if ftype is ctypes.c_void_p:
                if isinstance(v, str):          # LuaJIT points the field at the string's bytes
                    buf = ctypes.create_string_buffer(v.encode())
                    self.__dict__.setdefault("_strings", {})[k] = buf
                    setattr(st, k, ctypes.addressof(buf))
                else:
                    setattr(st, k, _to_addr(v))
            elif issubclass(ftype, ctypes.Array):
                setattr(st, k, v.encode() if isinstance(v, str) else v)
            else:
                n = v.v if isinstance(v, CInt64) else tonum(v)
                if n is None:
                    raise LuaError(f"cannot convert {lua_type(v)} to field '{k}'")
                setattr(st, k, n if ftype in _FLOATS else int(n))
            return
        et = self.ct.elem()
        i = int(k)
        if et.ptr:
            val = _to_addr(v)
        else:
            n = v.v if isinstance(v, CInt64) else tonum(v)
            if n is None:
                raise LuaError(f"cannot convert {lua_type(v)} to '{et.name}'")
            val = n if et.base in _FLOATS else int(n)
        if not self.is_pointer():
            self.obj[i] = val
        else:
            et.scalar_ctype().from_address(self.addr + i * et.size()).value = val

    def add(self, n):
        """Pointer arithmetic: a pointer, or an array decayed to one, plus n elements."""
        et = self.ct.elem()
        pt = CType(et.base, et.ptr + 1, et.name + "*")
        return CData(pt, addr=self.address() + int(n) * et.size())


_INT64_SIGNED = (ctypes.c_longlong, ctypes.c_int64, ctypes.c_long)
_INT64_UNSIGNED = (ctypes.c_ulonglong, ctypes.c_uint64, ctypes.c_ulong, ctypes.c_size_t)


def _from_c(v, ctype=None):
    if ctype is not None and ctypes.sizeof(ctype) == 8 and ctype in _INT64_SIGNED + _INT64_UNSIGNED:
        return CInt64(v, ctype in _INT64_UNSIGNED)
    if isinstance(v, bytes):
        return v.decode(errors="replace")
    if isinstance(v, (int, float)) and not isinstance(v, bool):
        return float(v)
    return v


def _to_addr(v):
    if v is None:
        return 0
    if isinstance(v, CData):
        return v.address()
    raise LuaError(f"cannot convert {lua_type(v)} to a pointer")


class FFI:
    def __init__(self):
        self.types = {}
        self.funcs = {}

    # -- declarations
    def parse_type(self, s):
        s = " ".join(s.replace("const ", "").split())
        vla = s.endswith("[?]")
        arrn = None
        if vla:
            s = s[:-3].strip()
        m = re.match(r"^(.*)\[(\d+)\]$", s)
        if m:
            s, arrn = m.group(1).strip(), int(m.group(2))
        ptr = s.count("*")
        base = s.replace("*", "").strip()
        if base in _CBASE:
            b = _CBASE[base]
        elif base in self.types:
            b = self.types[base]
        else:
            raise LuaError(f"ffi: unknown type '{base}'")
        name = base + "*" * ptr + ("[?]" if vla else f"[{arrn}]" if arrn is not None else "")
        return CType(b, ptr, name, vla, arrn)

    def cdef(self, text):
        text = re.sub(r"/\*.*?\*/|//[^\n]*", "", text, flags=re.S)
        for m in re.finditer(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", text, re.S):
            fields = []
            for decl in m.group(1).split(";"):
                decl = " ".join(decl.replace("const ", "").split())
                if not decl:
                    continue
                arr = re.match(r"^(.*?)\s+(\w+)\[(\d+)\]$", decl)
                if arr:
                    fields.append((arr.group(2), self.parse_type(arr.group(1)).scalar_ctype() * int(arr.group(3))))
                    continue
                head, names = re.match(r"^((?:unsigned\s+)?(?:long\s+long|\w+)\s*\**)\s*(.*)$", decl).groups()
                for nm in names.split(","):
                    nm = nm.strip()
                    t = self.parse_type(head + ("*" * nm.count("*")))
                    fields.append((nm.replace("*", "").strip(), t.scalar_ctype()))
            if m.group(2) in self.types:
                raise LuaError(f"attempt to redefine '{m.group(2)}'")
            self.types[m.group(2)] = type(m.group(2), (ctypes.Structure,), {"_fields_": fields})
        body = re.sub(r"typedef\s+struct\s*\{.*?\}\s*\w+\s*;", "", text, flags=re.S)
        for m in re.finditer(r"([\w\s\*]+?)\b(\w+)\s*\(([^;]*?)\)\s*;", body, re.S):
            ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
            args = []
            if params and params != "void":
                for prm in params.split(","):
                    prm = " ".join(prm.split())
                    pm = re.match(r"^(.*?[\s\*])(\w+)$", prm)
                    args.append(self.parse_type(pm.group(1) if pm else prm))
            if name in self.funcs:
                raise LuaError(f"attempt to redefine '{name}'")
            self.funcs[name] = (self.parse_type(ret), args)

    # -- objects
    def typeof(self, s):
        return self.parse_type(s)

    def new(self, ct, *init):
        if isinstance(ct, str):
            ct = self.parse_type(ct)
        return _ffi_new(ct, *init)

    def cast(self, ct, v):
        if isinstance(ct, str):
            ct = self.parse_type(ct)
        if ct.ptr and not ct.is_array():
            if isinstance(v, CInt64):
                return CData(ct, addr=v.v % (1 << 64))
            if isinstance(v, (int, float)) and not isinstance(v, bool):
                return CData(ct, addr=int(v))
            return CData(ct, addr=_to_addr(v))
        raise LuaError("ffi.cast: only pointer casts are supported here")

    def gc(self, cd, fin):
        old = getattr(cd, "_fin", None)
        if old is not None:
            old.detach()
        cd._fin = None
        if fin is not None:
            f = weakref.finalize(cd, _run_fin, fin, CData(cd.ct, addr=cd.address()))
            f.atexit = False
            cd._fin = f
        return cd

    def string(self, v, n=None):
        if isinstance(v, str):            # a char[] struct field reads back as text already
            return v if n is None else v[:int(n)]
        a = _to_addr(v)
        if n is not None:
            return ctypes.string_at(a, int(n)).decode(errors="replace")
        return ctypes.string_at(a).decode(errors="replace")


def _run_fin(fin, cd):
    try:
        fin(cd)
    except Exception:   # noqa: BLE001 -- finalisers must not raise
        pass


def _ffi_new(ct, *init):
    if ct.is_array():
        if ct.vla:
            if not init:
                raise LuaError("ffi.new: a variable-length array needs its size")
            n, init = int(init[0]), init[1:]
        else:
            n = ct.arrn
        et = ct.elem()
        arr = (et.scalar_ctype() * n)()
        cd = CData(CType(ct.base, ct.ptr, ct.name, ct.vla, n), obj=arr)
        for i, v in enumerate(init):
            cd.setindex(float(i), v)
        return cd
    if ct.ptr:
        return CData(ct, addr=_to_addr(init[0]) if init else 0)
    obj = ct.scalar_ctype()()
    if init and hasattr(obj, "value"):
        obj.value = init[0] if ct.base in _FLOATS else int(init[0])
    return CData(ct, obj=obj)


class CLib:
    def __init__(self, ffi, path):
        self.ffi = ffi
        try:
            self.lib = ctypes.CDLL(path)
        except OSError as ex:
            raise LuaError(f"cannot load library '{path}': {ex}") from None
        self.cache = {}

    def get(self, name):
        if name in self.cache:
            return self.cache[name]
        if name not in self.ffi.funcs:
            raise LuaError(f"missing declaration for symbol '{name}'")
        ret, args = self.ffi.funcs[name]
        fn = getattr(self.lib, name)
        void_ret = ret.ptr == 0 and ret.base is None
        fn.restype = None if void_ret else ret.scalar_ctype()
        fn.argtypes = [a.scalar_ctype() for a in args]

        def call(*vals):
            if len(vals) != len(args):
                raise LuaError(f"wrong number of arguments for function '{name}'")
            conv, keep = [], []
            for a, v in zip(args, vals):
                if a.ptr and isinstance(v, str):     # const char*: the string's bytes for the call
                    buf = ctypes.create_string_buffer(v.encode())
                    keep.append(buf)
                    conv.append(ctypes.addressof(buf))
                elif a.ptr:
                    conv.append(_to_addr(v))
                else:
                    n = v.v if isinstance(v, CInt64) else tonum(v)
                    if n is None:
                        raise LuaError(f"bad argument to '{name}': cannot convert {lua_type(v)} to a number")
                    conv.append(n if a.base in _FLOATS else int(n))
            r = fn(*conv)
            if void_ret:
                return None
            if ret.ptr:
                return CData(ret, addr=r or 0)
            return _from_c(r, ret.base)
        self.cache[name] = call
        return call


# ---------------------------------------------------------------- the interpreter
class LuaVM:
    def __init__(self):
        self.G = LuaTable()
        self.ffi = FFI()
        self.string_lib = LuaTable()
        self.loaded = LuaTable()
        self.search_dirs = []
        self.frames = []          # [short source, current line, chunk name] per running Lua function
        self._install_stdlib()

    # -- running code
    def load(self, text, chunkname="chunk"):
        ast = _AstParser(text, chunkname)
        block = ast.block()
        ast.expect("eof")
        return LuaFunction([], True, block, [], chunkname, self, chunkname)

    def dofile(self, path, *args):
        with open(path) as f:
            fn = self.load(f.read(), "@" + os.path.abspath(path))
        return self.call_function(fn, list(args))

    def call(self, f, *args):
        return self.call_value(f, list(args))

    def call_value(self, f, args):
        if isinstance(f, LuaFunction):
            return self.call_function(f, args)
        if isinstance(f, LuaTable):
            h = self.meta(f, "__call")
            if h is not None:
                return self.call_value(h, [f] + args)
            raise LuaError("attempt to call a table value")
        if isinstance(f, CType):
            return [f(*args)]
        if callable(f):
            r = f(*args)
            if r is None:
                return []
            if isinstance(r, tuple):
                return list(r)
            if isinstance(r, list):
                return r
            return [r]
        raise LuaError(f"attempt to call a {lua_type(f)} value")

    def _at(self, line):
        """Lua's position prefix for an error raised at `line` of the running function."""
        return f"{self.frames[-1][0]}:{int(line)}: " if self.frames else f"?:{int(line)}: "

    def call_function(self, fn, args):
        if len(self.frames) >= 190:
            raise LuaError("stack overflow")
        scope = {}
        for i, p in enumerate(fn.params):
            scope[p] = [args[i] if i < len(args) else None]
        if fn.vararg:
            scope["..."] = [args[len(fn.params):]]
        scopes = fn.scopes + [scope]
        self.frames.append([fn.src, 0, fn.chunk])
        try:
            self.exec_block(fn.body, scopes, new_scope=False)
        except _Return as r:
            return r.values
        finally:
            self.frames.pop()
        return []

    # -- metatables
    def meta(self, v, event):
        if isinstance(v, LuaTable):
            mt = v.meta
        elif isinstance(v, str):
            mt = self.string_meta
        else:
            return None
        return mt.rawget(event) if mt is not None else None

    def index(self, obj, key):
        if isinstance(obj, LuaTable):
            v = obj.rawget(key)
            if v is not None:
                return v
            h = self.meta(obj, "__index")
            if h is None:
                return None
            if isinstance(h, LuaTable):
                return self.index(h, key)
            return first(self.call_value(h, [obj, key]))
        if isinstance(obj, str):
            return self.string_lib.rawget(key)
        if isinstance(obj, CData):
            return obj.index(key)
        if isinstance(obj, CLib):
            return obj.get(key)
        if isinstance(obj, FFINamespace):
            return obj.get(key)
        raise LuaError(f"attempt to index a {lua_type(obj)} value")

    def setindex(self, obj, key, val):
        if isinstance(obj, LuaTable):
            if obj.rawget(key) is None:
                h = self.meta(obj, "__newindex")
                if h is not None:
                    if isinstance(h, LuaTable):
                        return self.setindex(h, key, val)
                    self.call_value(h, [obj, key, val])
                    return None
            obj.rawset(key, val)
            return None
        if isinstance(obj, CData):
            obj.setindex(key, val)
            return None
        raise LuaError(f"attempt to index a {lua_type(obj)} value")

    # -- statements
    def lookup(self, name, scopes):
        """The cell ([value]) of the innermost local `name`, or None for a global."""
        for s in reversed(scopes):
            c = s.get(name)
            if c is not None:
                return c
        return None

    def exec_block(self, block, scopes, new_scope=True):
        if new_scope:
            scopes = scopes + [{}]
        for st in block:
            self.exec_stat(st, scopes)

    def exec_stat(self, st, scopes):
        self.frames[-1][1] = st[-1]
        k = st[0]
        if k == "local":
            vals = self.eval_list(st[2], scopes)
            for i, nm in enumerate(st[1]):
                scopes[-1][nm] = [vals[i] if i < len(vals) else None]
        elif k == "assign":
            vals = self.eval_list(st[2], scopes)
            targets = []
            for t in st[1]:
                if t[0] == "name":
                    targets.append(("name", t[1]))
                else:
                    targets.append(("index", self.eval(t[1], scopes), self.eval(t[2], scopes)))
            for i, t in enumerate(targets):
                v = vals[i] if i < len(vals) else None
                if t[0] == "name":
                    c = self.lookup(t[1], scopes)
                    if c is not None:
                        c[0] = v
                    else:
                        self.G.rawset(t[1], v)
                else:
                    self.setindex(t[1], t[2], v)
        elif k == "callstat":
            self.eval_multi(st[1], scopes)
        elif k == "localfunc":
            cell = [None]
            scopes[-1][st[1]] = cell           # visible in its own body
            cell[0] = self.eval(st[2], scopes)
        elif k == "if":
            for cond, blk in st[1]:
                if truthy(self.eval(cond, scopes)):
                    self.exec_block(blk, scopes)
                    return
            if st[2] is not None:
                self.exec_block(st[2], scopes)
        elif k == "fornum":
            a = tonum(self.eval(st[2], scopes))
            b = tonum(self.eval(st[3], scopes))
            c = tonum(self.eval(st[4], scopes)) if st[4] is not None else 1.0
            if a is None or b is None or c is None:
                raise LuaError(self._at(st[6]) + f"'for' initial value, limit and step must be numbers")
            i = a
            try:
                while (c > 0 and i <= b) or (c <= 0 and i >= b):
                    self.exec_block(st[5], scopes + [{st[1]: [i]}], new_scope=False)
                    i += c
            except _Break:
                pass
        elif k == "forin":
            vals = self.eval_list(st[2], scopes)
            f, s, ctl = (vals + [None, None, None])[:3]
            try:
                while True:
                    rs = self.call_value(f, [s, ctl])
                    if not rs or rs[0] is None:
                        break
                    ctl = rs[0]
                    sc = {nm: [rs[i] if i < len(rs) else None] for i, nm in enumerate(st[1])}
                    self.exec_block(st[3], scopes + [sc], new_scope=False)
            except _Break:
                pass
        elif k == "while":
            try:
                while truthy(self.eval(st[1], scopes)):
                    self.exec_block(st[2], scopes)
            except _Break:
                pass
        elif k == "repeat":
            try:
                while True:
                    inner = scopes + [{}]
                    self.exec_block(st[1], inner, new_scope=False)
                    if truthy(self.eval(st[2], inner)):
                        break
            except _Break:
                pass
        elif k == "do":
            self.exec_block(st[1], scopes)
        elif k == "return":
            raise _Return(self.eval_list(st[1], scopes))
        elif k == "break":
            raise _Break()
        else:
            raise LuaError(f"unsupported statement {k}")

    # -- expressions
    def eval_list(self, exprs, scopes):
        out = []
        for i, e in enumerate(exprs):
            if i == len(exprs) - 1:
                out.extend(self.eval_multi(e, scopes))
            else:
                out.append(self.eval(e, scopes))
        return out

    def eval_multi(self, e, scopes):
        k = e[0]
        if k == "call":
            f = self.eval(e[1], scopes)
            args = self.eval_list(e[2], scopes)
            return self._call_at(f, args, e)
        if k == "method":
            obj = self.eval(e[1], scopes)
            f = self.index(obj, e[2])
            args = [obj] + self.eval_list(e[3], scopes)
            return self._call_at(f, args, e)
        if k == "vararg":
            c = self.lookup("...", scopes)
            return list(c[0]) if c is not None else []
        return [self.eval(e, scopes)]

    def _call_at(self, f, args, e):
        if f is None:
            what = e[1][1] if e[0] == "call" and e[1][0] == "name" else (e[2] if e[0] == "method" else "?")
            raise LuaError(self._at(e[-1]) + f"attempt to call a nil value ({what})")
        return self.call_value(f, args)

    def eval(self, e, scopes):
        k = e[0]
        if k == "num" or k == "str":
            return e[1]
        if k == "name":
            c = self.lookup(e[1], scopes)
            return c[0] if c is not None else self.G.rawget(e[1])
        if k == "index":
            obj = self.eval(e[1], scopes)
            if obj is None:
                raise LuaError(self._at(e[3]) + f"attempt to index a nil value")
            return self.index(obj, self.eval(e[2], scopes))
        if k in ("call", "method", "vararg"):
            return first(self.eval_multi(e, scopes))
        if k == "nil":
            return None
        if k == "true":
            return True
        if k == "false":
            return False
        if k == "paren":
            return self.eval(e[1], scopes)
        if k == "and":
            a = self.eval(e[1], scopes)
            return self.eval(e[2], scopes) if truthy(a) else a
        if k == "or":
            a = self.eval(e[1], scopes)
            return a if truthy(a) else self.eval(e[2], scopes)
        if k == "bin":
            return self.binop(e[1], self.eval(e[2], scopes), self.eval(e[3], scopes), e[4])
        if k == "un":
            v = self.eval(e[2], scopes)
            if e[1] == "not":
                return not truthy(v)
            if e[1] == "-" and isinstance(v, CInt64):
                return CInt64(-v.v, v.unsigned)
            if e[1] == "-":
                n = tonum(v)
                if n is None:
                    raise LuaError(self._at(e[3]) + f"attempt to perform arithmetic on a {lua_type(v)} value")
                return -n
            if isinstance(v, str):
                return float(len(v.encode()))
            if isinstance(v, LuaTable):
                return float(v.length())
            raise LuaError(self._at(e[3]) + f"attempt to get length of a {lua_type(v)} value")
        if k == "table":
            t = LuaTable()
            pos = 1
            items = e[1]
            for i, (kind, key, val) in enumerate(items):
                if kind == "pos":
                    if i == len(items) - 1:
                        for v in self.eval_multi(val, scopes):
                            t.rawset(float(pos), v)
                            pos += 1
                    else:
                        t.rawset(float(pos), self.eval(val, scopes))
                        pos += 1
                else:
                    t.rawset(self.eval(key, scopes), self.eval(val, scopes))
            return t
        if k == "func":
            # upvalues: the cells of the locals the body names, as visible now
            up = {}
            for nm in e[6]:
                c = self.lookup(nm, scopes)
                if c is not None:
                    up[nm] = c
            return LuaFunction(e[1], e[2], e[3], [up], e[4], self, e[7])
        raise LuaError(f"unsupported expression {k}")

    def binop(self, op, a, b, line):
        if op == "..":
            if isinstance(a, (str, int, float)) and isinstance(b, (str, int, float)) and \
                    not isinstance(a, bool) and not isinstance(b, bool):
                return tostr(a) + tostr(b)
            raise LuaError(self._at(line) + f"attempt to concatenate a {lua_type(b if isinstance(a, (str, float)) else a)} value")
        if op == "==":
            return lua_eq(a, b)
        if op == "~=":
            return not lua_eq(a, b)
        if isinstance(a, CInt64) or isinstance(b, CInt64):
            return self.int64_op(op, a, b, line)
        if op in ("<", ">", "<=", ">="):
            if isinstance(a, str) and isinstance(b, str):
                pass
            elif not (isinstance(a, (int, float)) and isinstance(b, (int, float))) or isinstance(a, bool) \
                    or isinstance(b, bool):
                raise LuaError(self._at(line) + f"attempt to compare {lua_type(a)} with {lua_type(b)}")
            return {"<": a < b, ">": a > b, "<=": a <= b, ">=": a >= b}[op]
        if op == "+" and isinstance(a, CData):
            return a.add(tonum(b))
        x, y = tonum(a), tonum(b)
        if x is None or y is None:
            bad = a if x is None else b
            raise LuaError(self._at(line) + f"attempt to perform arithmetic on a {lua_type(bad)} value")
        if op == "+":
            return x + y
        if op == "-":
            return x - y
        if op == "*":
            return x * y
        if op == "/":
            if y == 0:
                return math.copysign(math.inf, x) * math.copysign(1, y) if x != 0 else math.nan
            return x / y
        if op == "%":
            if y == 0:
                return math.nan
            return x - math.floor(x / y) * y
        if op == "^":
            return math.pow(x, y)
        raise LuaError(self._at(line) + f"unsupported operator {op}")

    def int64_op(self, op, a, b, line):
        """+ - * and comparisons with a 64-bit integer cdata operand (the other
        a number or one too): the result is 64-bit, unsigned if either is."""
        def val(x):
            if isinstance(x, CInt64):
                return x.v
            if isinstance(x, (int, float)) and not isinstance(x, bool):
                return int(x)
            raise LuaError(self._at(line) + f"attempt to perform arithmetic on a {lua_type(x)} value")
        if isinstance(a, CData):      # pointer + int64
            if op == "+":
                return a.add(val(b))
            raise LuaError(self._at(line) + "attempt to perform arithmetic on a cdata value")
        x, y = val(a), val(b)
        uns = any(isinstance(t, CInt64) and t.unsigned for t in (a, b))
        if op in ("<", ">", "<=", ">="):
            return {"<": x < y, ">": x > y, "<=": x <= y, ">=": x >= y}[op]
        if op == "+":
            return CInt64(x + y, uns)
        if op == "-":
            return CInt64(x - y, uns)
        if op == "*":
            return CInt64(x * y, uns)
        raise LuaError(self._at(line) + f"operator {op} on a 64-bit integer cdata is not supported here")

    # -- standard library (the parts the files use)
    def _install_stdlib(self):
        G = self.G
        vm = self

        def lua_error(msg=None, level=1.0):
            lvl = int(level)
            if isinstance(msg, str) and 0 < lvl <= len(vm.frames):
                src, line = vm.frames[-lvl][:2]
                msg = f"{src}:{int(line)}: {msg}"
            raise LuaError(msg)

        def lua_pcall(f, *args):
            try:
                return [True] + vm.call_value(f, list(args))
            except LuaError as ex:
                return [False, ex.value]
            except (_Break, _Return):
                raise
            except Exception as ex:  # noqa: BLE001 -- a Python-side failure is a Lua error
                return [False, f"{type(ex).__name__}: {ex}"]

        def lua_select(n, *args):
            if n == "#":
                return float(len(args))
            i = int(n)
            return list(args[i - 1:]) if i > 0 else list(args[i:])

        def lua_ipairs(t):
            if not isinstance(t, LuaTable):
                raise LuaError(f"bad argument #1 to 'ipairs' (table expected, got {lua_type(t)})")

            def it(t_, i):
                i = int(i) + 1
                v = vm.index(t_, float(i))
                return None if v is None else [float(i), v]
            return [it, t, 0.0]

        def lua_next(t, k=None):
            keys = list(t.d.keys())
            if k is None:
                idx = 0
            else:
                kk = LuaTable.key(k)
                if kk not in t.d:
                    raise LuaError("invalid key to 'next'")
                idx = keys.index(kk) + 1
            if idx >= len(keys):
                return [None]
            key = keys[idx]
            return [_lua_key(key), t.d[key]]

        def lua_pairs(t):
            if not isinstance(t, LuaTable):
                raise LuaError(f"bad argument #1 to 'pairs' (table expected, got {lua_type(t)})")
            keys = list(t.d.keys())
            pos = [0]

            def it(_s, _c):
                while pos[0] < len(keys):
                    k = keys[pos[0]]
                    pos[0] += 1
                    if k in t.d:
                        return [_lua_key(k), t.d[k]]
                return None
            return [it, t, None]

        def lua_setmetatable(t, mt):
            t.meta = mt
            return t

        def lua_getmetatable(t):
            return [t.meta if isinstance(t, LuaTable) else None]

        def lua_tostring(v):
            return tostr(v)

        def lua_tonumber(v, base=None):
            if isinstance(v, CInt64):
                return [float(v.v)]
            if base is not None:
                try:
                    return [float(int(str(v).strip(), int(base)))]
                except ValueError:
                    return [None]
            return [tonum(v)]

        def lua_require(name):
            v = vm.loaded.rawget(name)
            if v is not None:
                return v
            if name == "ffi":
                return vm.ffi_ns
            for d in vm.search_dirs:
                p = os.path.join(d, name.replace(".", "/") + ".lua")
                if os.path.exists(p):
                    r = first(vm.dofile(p))
                    r = True if r is None else r
                    vm.loaded.rawset(name, r)
                    return r
            raise LuaError(f"module '{name}' not found")

        def lua_assert(v, msg=None, *rest):
            if not truthy(v):
                raise LuaError(msg if msg is not None else "assertion failed!")
            return [v, msg] + list(rest)

        for nm, fn in {"error": lua_error, "pcall": lua_pcall, "select": lua_select, "ipairs": lua_ipairs,
                       "pairs": lua_pairs, "next": lua_next, "setmetatable": lua_setmetatable,
                       "getmetatable": lua_getmetatable, "tostring": lua_tostring, "tonumber": lua_tonumber,
                       "type": lua_type, "require": lua_require, "assert": lua_assert,
                       "rawequal": lambda a, b: a is b or (a == b and type(a) is type(b)),
                       "rawget": lambda t, k: [t.rawget(k)], "rawset": lambda t, k, v: (t.rawset(k, v), t)[1],
                       "unpack": lambda t, i=1.0, j=None: [t.rawget(float(x)) for x in
                                                           range(int(i), int(j if j is not None else t.length()) + 1)], "print": lambda *a: print(*[tostr(x) for x in a])
                       }.items():
            G.rawset(nm, fn)

        # string
        S = self.string_lib

        def s_format(fmt, *args):
            out, ai, i = [], 0, 0
            while i < len(fmt):
                c = fmt[i]
                if c != "%":
                    out.append(c)
                    i += 1
                    continue
                m = re.match(r"%([-+ #0]*\d*(?:\.\d+)?)([diouxXeEfgGqsc%])", fmt[i:])
                if not m:
                    raise LuaError(f"invalid format {fmt[i:i + 4]!r}")
                spec, conv = m.groups()
                i += m.end()
                if conv == "%":
                    out.append("%")
                    continue
                v = args[ai] if ai < len(args) else None
                ai += 1
                if conv in "dioxXuc":
                    n = v.v if isinstance(v, CInt64) else tonum(v)
                    if n is None:
                        raise LuaError(f"bad argument #{ai} to 'format' (number expected, got {lua_type(v)})")
                    out.append(("%" + spec + ("d" if conv in "iu" else conv)) % int(n) if conv != "c"
                               else chr(int(n)))
                elif conv in "eEfgG":
                    n = tonum(v)
                    if n is None:
                        raise LuaError(f"bad argument #{ai} to 'format' (number expected, got {lua_type(v)})")
                    out.append(("%" + spec + conv) % n)
                elif conv == "q":
                    out.append('"' + tostr(v).replace("\\", "\\\\").replace('"', '\\"') + '"')
                else:
                    if not isinstance(v, (str, int, float)) or isinstance(v, bool):
                        raise LuaError(f"bad argument #{ai} to 'format' (string expected, got {lua_type(v)})")
                    out.append(("%" + spec + "s") % tostr(v))
            return "".join(out)

        def s_sub(s, i=1.0, j=-1.0):
            n = len(s)
            i, j = int(i), int(j)
            if i < 0:
                i = max(n + i + 1, 1)
            elif i == 0:
                i = 1
            if j < 0:
                j = n + j + 1
            elif j > n:
                j = n
            return s[i - 1:j] if i <= j else ""

        def s_match(s, pat, init=1.0):
            m = re.compile(lua_pattern_to_re(pat), re.S).search(s, int(init) - 1)
            if not m:
                return [None]
            return list(m.groups()) if m.groups() else [m.group(0)]

        def s_find(s, pat, init=1.0, plain=None):
            start = int(init) - 1
            if truthy(plain):
                j = s.find(pat, start)
                return [None] if j < 0 else [float(j + 1), float(j + len(pat))]
            m = re.compile(lua_pattern_to_re(pat), re.S).search(s, start)
            if not m:
                return [None]
            return [float(m.start() + 1), float(m.end())] + list(m.groups())

        def s_rep(s, n, sep=""):
            return sep.join([s] * int(n))

        for nm, fn in {"format": s_format, "sub": s_sub, "match": s_match, "find": s_find, "rep": s_rep,
                       "len": lambda s: float(len(s)), "upper": lambda s: s.upper(),
                       "lower": lambda s: s.lower(), "byte": lambda s, i=1.0: float(ord(s[int(i) - 1])),
                       "char": lambda *c: "".join(chr(int(x)) for x in c)}.items():
            S.rawset(nm, fn)
        G.rawset("string", S)
        self.string_meta = LuaTable()
        self.string_meta.rawset("__index", S)

        # table, math, os, debug
        T = LuaTable()
        T.rawset("insert", lambda t, *a: t.rawset(float(t.length() + 1), a[0]) if len(a) == 1 else _tinsert(t, *a))
        T.rawset("concat", lambda t, sep="", i=1.0, j=None: sep.join(
            tostr(t.rawget(float(k))) for k in range(int(i), int(j if j is not None else t.length()) + 1)))
        T.rawset("remove", lambda t, pos=None: _tremove(t, pos))
        G.rawset("table", T)
        Mth = LuaTable()
        for nm, fn in {"max": lambda *a: max(a), "min": lambda *a: min(a), "floor": lambda x: float(math.floor(x)),
                       "ceil": lambda x: float(math.ceil(x)), "sqrt": math.sqrt, "abs": abs, "exp": math.exp,
                       "log": lambda x, b=None: math.log(x) if b is None else math.log(x, b),
                       "fmod": math.fmod}.items():
            Mth.rawset(nm, fn)
        Mth.rawset("huge", math.inf)
        Mth.rawset("pi", math.pi)
        G.rawset("math", Mth)
        Os = LuaTable()
        Os.rawset("getenv", lambda k: [os.environ.get(k)])
        Os.rawset("clock", lambda: __import__("time").process_time())
        G.rawset("os", Os)
        Dbg = LuaTable()

        def d_getinfo(level=1.0, what=""):
            lvl = int(level)
            if not 0 < lvl <= len(vm.frames):
                return [None]
            fr = vm.frames[-lvl]
            info = LuaTable()
            info.rawset("source", fr[2])
            info.rawset("short_src", fr[0])
            info.rawset("currentline", float(fr[1]))
            return info
        Dbg.rawset("getinfo", d_getinfo)
        G.rawset("debug", Dbg)
        self.ffi_ns = FFINamespace(self)


def _tinsert(t, pos, v):
    n = t.length()
    for i in range(n, int(pos) - 1, -1):
        t.rawset(float(i + 1), t.rawget(float(i)))
    t.rawset(float(pos), v)


def _tremove(t, pos=None):
    n = t.length()
    if n == 0:
        return None
    pos = n if pos is None else int(pos)
    v = t.rawget(float(pos))
    for i in range(pos, n):
        t.rawset(float(i), t.rawget(float(i + 1)))
    t.rawset(float(n), None)
    return v


class FFINamespace:
    """The ``ffi`` module table seen from Lua."""

    def __init__(self, vm):
        self.vm = vm
        f = vm.ffi
        self.fns = {
            "cdef": lambda text: f.cdef(text),
            "load": lambda path: CLib(f, path),
            "new": f.new, "typeof": f.typeof, "cast": f.cast, "gc": f.gc, "string": f.string,
        }

    def get(self, k):
        if k in self.fns:
            return self.fns[k]
        raise LuaError(f"ffi.{k} is not supported by this interpreter")


def _lua_key(k):
    return float(k) if isinstance(k, int) and not isinstance(k, bool) else k


def first(vals):
    return vals[0] if vals else None


def lua_eq(a, b):
    if a is None or b is None:
        if isinstance(a, CData) and a.is_pointer():
            return a.addr == 0 and b is None
        if isinstance(b, CData) and b.is_pointer():
            return b.addr == 0 and a is None
        return a is b
    if isinstance(a, bool) or isinstance(b, bool):
        return a is b
    if isinstance(a, (int, float)) and isinstance(b, (int, float)):
        return float(a) == float(b)
    if isinstance(a, CInt64) or isinstance(b, CInt64):
        def iv(x):
            if isinstance(x, CInt64):
                return x.v
            return x if isinstance(x, (int, float)) else None
        x, y = iv(a), iv(b)
        return x is not None and y is not None and x == y
    if isinstance(a, str) and isinstance(b, str):
        return a == b
    if isinstance(a, CData) and isinstance(b, CData) and a.is_pointer() and b.is_pointer():
        return a.addr == b.addr
    return a is b


def run_module(path, vm=None):
    """Run a Lua file as ``require`` would and return (vm, its first result)."""
    vm = vm or LuaVM()
    r = first(vm.dofile(path))
    return vm, r
