"""A Lua 5.1 / LuaJIT parser and scope resolver, used by the CPU tests to check
lanternl_amd/lua/luatl_adapter.lua without a Lua runtime (none exists in this
image or on the GPU box).

* ``parse(text)`` tokenizes and parses the whole chunk by the Lua 5.1 grammar
  (plus LuaJIT's ``goto`` and ``::label::``), raising ``LuaSyntaxError`` with
  the line of the first error.
* ``free_names(text)`` resolves every name against the lexical scopes the
  grammar defines (``local``, ``local function``, function parameters, loop
  variables, ``self`` in ``function a:b()``) and returns the names read or
  written as globals, with the line of their first use.  A name used above
  its ``local`` declaration, or a misspelt local, shows up there.

Test infrastructure only: it checks the Lua text, it runs nothing.
"""
import re


class LuaSyntaxError(Exception):
    pass


KEYWORDS = {"and", "break", "do", "else", "elseif", "end", "false", "for", "function", "goto", "if", "in",
            "local", "nil", "not", "or", "repeat", "return", "then", "true", "until", "while"}
OPS3 = {"..."}
OPS2 = {"==", "~=", "<=", ">=", "..", "::"}
OPS1 = set("+-*/%^#<>=(){}[];:,.")

BINPRI = {"or": (1, 1), "and": (2, 2), "<": (3, 3), ">": (3, 3), "<=": (3, 3), ">=": (3, 3), "~=": (3, 3),
          "==": (3, 3), "..": (5, 4), "+": (6, 6), "-": (6, 6), "*": (7, 7), "/": (7, 7), "%": (7, 7),
          "^": (10, 9)}
UNARY_PRI = 8


def tokenize(text):
    """[(kind, value, line)]: kind is 'name', 'kw', 'num', 'str', 'op' or 'eof'.
    A 'str' token carries a fourth field: True for a long bracket string (its
    text raw), False for a quoted one (its text with the escapes unprocessed)."""
    toks, i, line, n = [], 0, 1, len(text)
    while i < n:
        c = text[i]
        if c == "\n":
            line += 1
            i += 1
            continue
        if c in " \t\r\f\v":
            i += 1
            continue
        if text.startswith("--", i):
            m = re.match(r"--\[(=*)\[", text[i:])
            if m:
                close = "]" + m.group(1) + "]"
                j = text.find(close, i + m.end())
                if j < 0:
                    raise LuaSyntaxError(f"line {line}: unfinished long comment")
                line += text.count("\n", i, j)
                i = j + len(close)
            else:
                j = text.find("\n", i)
                i = n if j < 0 else j
            continue
        m = re.match(r"\[(=*)\[", text[i:])
        if m:
            close = "]" + m.group(1) + "]"
            j = text.find(close, i + m.end())
            if j < 0:
                raise LuaSyntaxError(f"line {line}: unfinished long string")
            toks.append(("str", text[i + m.end():j], line, True))
            line += text.count("\n", i, j)
            i = j + len(close)
            continue
        if c in "\"'":
            j = i + 1
            while True:
                if j >= n or text[j] == "\n":
                    raise LuaSyntaxError(f"line {line}: unfinished string")
                if text[j] == "\\":
                    if j + 1 < n and text[j + 1] == "\n":
                        line += 1
                    j += 2
                    continue
                if text[j] == c:
                    break
                j += 1
            toks.append(("str", text[i + 1:j], line, False))
            i = j + 1
            continue
        m = re.match(r"0[xX][0-9a-fA-F]+(?:[uU]?[lL][lL])?|(?:\d+\.?\d*|\.\d+)(?:[eE][+-]?\d+)?(?:[uU]?[lL][lL]|i)?",
                     text[i:])
        if m and m.group(0) and (c.isdigit() or (c == "." and i + 1 < n and text[i + 1].isdigit())):
            toks.append(("num", m.group(0), line))
            i += m.end()
            continue
        m = re.match(r"[A-Za-z_][A-Za-z0-9_]*", text[i:])
        if m:
            w = m.group(0)
            toks.append(("kw" if w in KEYWORDS else "name", w, line))
            i += m.end()
            continue
        for ops in (OPS3, OPS2, OPS1):
            w = text[i:i + len(next(iter(ops)))]
            if w in ops:
                toks.append(("op", w, line))
                i += len(w)
                break
        else:
            raise LuaSyntaxError(f"line {line}: unexpected character {c!r}")
    toks.append(("eof", "<eof>", line))
    return toks


class _Parser:
    """Recursive descent over the Lua 5.1 grammar, resolving names as it goes."""

    def __init__(self, text):
        self.t = tokenize(text)
        self.p = 0
        self.scopes = [set()]
        self.free = {}

    # -- tokens
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
            raise LuaSyntaxError(f"line {tk[2]}: expected {value or kind}, got {tk[1]!r}")
        self.p += 1
        return tk

    def name(self):
        return self.expect("name")[1]

    # -- scopes
    def push(self):
        self.scopes.append(set())

    def pop(self):
        self.scopes.pop()

    def declare(self, nm):
        self.scopes[-1].add(nm)

    def use(self, nm, line):
        if not any(nm in s for s in self.scopes):
            self.free.setdefault(nm, line)

    # -- blocks
    def block_follow(self):
        tk = self.peek()
        return tk[0] == "eof" or (tk[0] == "kw" and tk[1] in ("else", "elseif", "end", "until"))

    def block(self):
        while not self.block_follow():
            if self.check("kw", "return"):
                self.p += 1
                if not self.block_follow() and not self.check("op", ";"):
                    self.explist()
                self.accept("op", ";")
                break
            if self.check("kw", "break"):
                self.p += 1
                self.accept("op", ";")
                continue
            self.statement()
            self.accept("op", ";")

    def scoped_block(self):
        self.push()
        self.block()
        self.pop()

    def statement(self):
        tk = self.peek()
        if tk[0] == "kw":
            kw = tk[1]
            if kw == "do":
                self.p += 1
                self.scoped_block()
                self.expect("kw", "end")
                return
            if kw == "while":
                self.p += 1
                self.expr()
                self.expect("kw", "do")
                self.scoped_block()
                self.expect("kw", "end")
                return
            if kw == "repeat":
                self.p += 1
                self.push()
                self.block()
                self.expect("kw", "until")
                self.expr()              # the condition sees the body's locals
                self.pop()
                return
            if kw == "if":
                self.p += 1
                self.expr()
                self.expect("kw", "then")
                self.scoped_block()
                while self.accept("kw", "elseif"):
                    self.expr()
                    self.expect("kw", "then")
                    self.scoped_block()
                if self.accept("kw", "else"):
                    self.scoped_block()
                self.expect("kw", "end")
                return
            if kw == "for":
                self.p += 1
                first = self.name()
                if self.accept("op", "="):
                    self.expr()
                    self.expect("op", ",")
                    self.expr()
                    if self.accept("op", ","):
                        self.expr()
                    names = [first]
                else:
                    names = [first]
                    while self.accept("op", ","):
                        names.append(self.name())
                    self.expect("kw", "in")
                    self.explist()
                self.expect("kw", "do")
                self.push()
                for nm in names:
                    self.declare(nm)
                self.block()
                self.pop()
                self.expect("kw", "end")
                return
            if kw == "function":
                self.p += 1
                line = self.peek()[2]
                nm = self.name()
                self.use(nm, line)
                method = False
                while self.check("op", ".") or self.check("op", ":"):
                    method = self.peek()[1] == ":"
                    self.p += 1
                    self.name()
                    if method:
                        break
                self.funcbody(method)
                return
            if kw == "local":
                self.p += 1
                if self.accept("kw", "function"):
                    nm = self.name()
                    self.declare(nm)     # visible inside its own body (recursion)
                    self.funcbody(False)
                    return
                names = [self.name()]
                while self.accept("op", ","):
                    names.append(self.name())
                if self.accept("op", "="):
                    self.explist()       # the values do not see the new locals
                for nm in names:
                    self.declare(nm)
                return
            if kw == "goto":
                self.p += 1
                self.name()
                return
        if self.accept("op", "::"):
            self.name()
            self.expect("op", "::")
            return
        # exprstat: a call, or an assignment to a variable list
        kind = self.suffixedexp()
        if self.check("op", "=") or self.check("op", ","):
            if kind != "var":
                raise LuaSyntaxError(f"line {self.peek()[2]}: cannot assign to this expression")
            while self.accept("op", ","):
                if self.suffixedexp() != "var":
                    raise LuaSyntaxError(f"line {self.peek()[2]}: cannot assign to this expression")
            self.expect("op", "=")
            self.explist()
        elif kind != "call":
            raise LuaSyntaxError(f"line {self.peek()[2]}: syntax error near {self.peek()[1]!r}")

    def funcbody(self, method):
        self.expect("op", "(")
        self.push()
        if method:
            self.declare("self")
        if not self.check("op", ")"):
            while True:
                if self.accept("op", "..."):
                    break
                self.declare(self.name())
                if not self.accept("op", ","):
                    break
        self.expect("op", ")")
        self.block()
        self.pop()
        self.expect("kw", "end")

    # -- expressions
    def explist(self):
        self.expr()
        while self.accept("op", ","):
            self.expr()

    def primaryexp(self):
        tk = self.peek()
        if tk[0] == "name":
            self.p += 1
            self.use(tk[1], tk[2])
            return "var"
        if self.accept("op", "("):
            self.expr()
            self.expect("op", ")")
            return "paren"
        raise LuaSyntaxError(f"line {tk[2]}: unexpected symbol {tk[1]!r}")

    def suffixedexp(self):
        kind = self.primaryexp()
        while True:
            if self.accept("op", "."):
                self.name()
                kind = "var"
            elif self.accept("op", "["):
                self.expr()
                self.expect("op", "]")
                kind = "var"
            elif self.accept("op", ":"):
                self.name()
                self.callargs()
                kind = "call"
            elif self.check("op", "(") or self.check("op", "{") or self.check("str"):
                self.callargs()
                kind = "call"
            else:
                return kind

    def callargs(self):
        if self.accept("str"):
            return
        if self.check("op", "{"):
            self.table()
            return
        self.expect("op", "(")
        if not self.check("op", ")"):
            self.explist()
        self.expect("op", ")")

    def table(self):
        self.expect("op", "{")
        while not self.check("op", "}"):
            if self.accept("op", "["):
                self.expr()
                self.expect("op", "]")
                self.expect("op", "=")
                self.expr()
            elif self.check("name") and self.peek(1)[0] == "op" and self.peek(1)[1] == "=":
                self.p += 2
                self.expr()
            else:
                self.expr()
            if not (self.accept("op", ",") or self.accept("op", ";")):
                break
        self.expect("op", "}")

    def simpleexp(self):
        tk = self.peek()
        if tk[0] in ("num", "str"):
            self.p += 1
        elif tk[0] == "kw" and tk[1] in ("nil", "true", "false"):
            self.p += 1
        elif self.accept("op", "..."):
            pass
        elif self.check("op", "{"):
            self.table()
        elif self.accept("kw", "function"):
            self.funcbody(False)
        else:
            self.suffixedexp()

    def expr(self, limit=0):
        tk = self.peek()
        if (tk[0] == "kw" and tk[1] == "not") or (tk[0] == "op" and tk[1] in ("-", "#")):
            self.p += 1
            self.expr(UNARY_PRI)
        else:
            self.simpleexp()
        while True:
            tk = self.peek()
            op = tk[1] if tk[0] in ("op", "kw") else None
            if op not in BINPRI or BINPRI[op][0] <= limit:
                return
            self.p += 1
            self.expr(BINPRI[op][1])


def parse(text):
    """Parse a whole chunk; raises LuaSyntaxError on the first error."""
    ps = _Parser(text)
    ps.block()
    ps.expect("eof")
    return ps


def free_names(text):
    """{name: first line} of every name resolved to no enclosing local."""
    return dict(parse(text).free)
