"""A reader for the Common Lisp syntax llambda's sources and INTEGRATION.md's
Lisp blocks use, and the names those forms define or call.

Only what a name check needs: lists, strings, characters, numbers, symbols
(folded to lower case, package prefixes kept), quote / backquote / comma,
#' #P #x #. #: #+ #- and comments.  Used by tests/golden/make_reference_symbols.py
(the names the reference defines) and tests/test_integration_lisp.py (the
names the adapter code calls)."""
from __future__ import annotations

import re
from typing import Iterator, List, Set


class Sym(str):
    """A symbol, lower-cased; keywords keep their leading colon."""


class Str(str):
    """A string literal."""


def _quoted(kind: str, form):
    return [Sym(kind), form]


_DELIMS = set("()'`,\";")
_NUMBER = re.compile(r"^[+-]?(\d+\.?\d*([edfs][+-]?\d+)?|\.\d+([edfs][+-]?\d+)?|\d+/\d+)$", re.I)


class Reader:
    def __init__(self, text: str):
        self.s = text
        self.i = 0

    def _skip(self):
        s, n = self.s, len(self.s)
        while self.i < n:
            c = s[self.i]
            if c.isspace():
                self.i += 1
            elif c == ";":
                j = s.find("\n", self.i)
                self.i = n if j < 0 else j + 1
            elif s.startswith("#|", self.i):
                depth, self.i = 1, self.i + 2
                while depth and self.i < n:
                    if s.startswith("|#", self.i):
                        depth, self.i = depth - 1, self.i + 2
                    elif s.startswith("#|", self.i):
                        depth, self.i = depth + 1, self.i + 2
                    else:
                        self.i += 1
            else:
                return

    def forms(self) -> Iterator:
        while True:
            self._skip()
            if self.i >= len(self.s):
                return
            yield self.read()

    def _token(self) -> str:
        s, n, j = self.s, len(self.s), self.i
        while j < n and not s[j].isspace() and s[j] not in _DELIMS:
            j += 1
        tok, self.i = s[self.i:j], j
        return tok

    def read(self):
        self._skip()
        if self.i >= len(self.s):
            raise EOFError("end of input inside a form")
        s = self.s
        c = s[self.i]
        if c == "(":
            self.i += 1
            out: List = []
            while True:
                self._skip()
                if self.i >= len(s):
                    raise EOFError("unclosed list")
                if s[self.i] == ")":
                    self.i += 1
                    return out
                if s[self.i] == "." and (self.i + 1 < len(s)) and s[self.i + 1].isspace():
                    self.i += 1  # dotted pair: keep the tail as the last element
                    continue
                out.append(self.read())
        if c == ")":
            raise SyntaxError(f"unexpected ')' at offset {self.i}")
        if c == "'":
            self.i += 1
            return _quoted("quote", self.read())
        if c == "`":
            self.i += 1
            return _quoted("quasiquote", self.read())
        if c == ",":
            self.i += 1
            if self.i < len(s) and s[self.i] in "@.":
                self.i += 1
            return _quoted("unquote", self.read())
        if c == '"':
            j, buf = self.i + 1, []
            while s[j] != '"':
                if s[j] == "\\":
                    j += 1
                buf.append(s[j])
                j += 1
            self.i = j + 1
            return Str("".join(buf))
        if c == "#":
            d = s[self.i + 1]
            if d == "'":
                self.i += 2
                return _quoted("function", self.read())
            if d == "\\":
                start = self.i + 2
                j = start + 1  # the character itself, then any name letters
                while j < len(s) and (s[j].isalnum() or s[j] in "-_"):
                    j += 1
                self.i = j
                return Str(s[start:j])  # a character: data, never a name
            if d in "Pp":
                self.i += 2
                return self.read()
            if d in "xXbBoO":
                self.i += 2
                return int(self._token(), {"x": 16, "b": 2, "o": 8}[d.lower()])
            if d == ".":
                self.i += 2
                return _quoted("read-eval", self.read())
            if d == ":":
                self.i += 2
                return Sym("#:" + self._token().lower())
            if d in "+-":
                self.i += 2
                feature = self.read()
                form = self.read()
                return _quoted("feature-" + d, [feature, form])
            if d == "(":
                self.i += 1
                return _quoted("vector", self.read())
            raise SyntaxError(f"unsupported dispatch #{d} at offset {self.i}")
        tok = self._token()
        if not tok:
            raise SyntaxError(f"empty token at offset {self.i}")
        if _NUMBER.match(tok):
            return tok  # numbers stay text: the name checks never look at them
        return Sym(tok.lower())


def read_all(text: str) -> list:
    return list(Reader(text).forms())


# ------------------------------------------------------------- definitions

def _name(x) -> str:
    return x if isinstance(x, Sym) else ""


def struct_names(form) -> Set[str]:
    """Every function a defstruct defines: constructor(s), predicate, copier and
    slot accessors, with :conc-name / :constructor / :predicate / :copier."""
    spec = form[1]
    opts = []
    if isinstance(spec, list):
        name, opts = _name(spec[0]), spec[1:]
    else:
        name = _name(spec)
    conc, ctors, pred, copier = name + "-", [], name + "-p", "copy-" + name
    explicit_ctor = False
    for o in opts:
        key = o[0] if isinstance(o, list) else o
        args = o[1:] if isinstance(o, list) else []
        if key == ":conc-name":
            conc = (str(args[0]) if args and args[0] not in ("nil",) else "") if args else ""
        elif key == ":constructor":
            explicit_ctor = True
            if args and args[0] != "nil":
                ctors.append(str(args[0]))
        elif key == ":predicate":
            pred = str(args[0]) if args and args[0] != "nil" else ""
        elif key == ":copier":
            copier = str(args[0]) if args and args[0] != "nil" else ""
    if not explicit_ctor:
        ctors.append("make-" + name)
    out = {n for n in ctors + [pred, copier] if n}
    body = form[2:]
    if body and isinstance(body[0], Str):
        body = body[1:]
    for slot in body:
        slot_name = _name(slot[0] if isinstance(slot, list) else slot)
        if slot_name:
            out.add(conc + slot_name)
    return out


DEFINERS_FUNCTION = {"defun", "defmacro", "defgeneric", "defmethod"}
DEFINERS_VARIABLE = {"defvar", "defparameter", "defconstant"}


def defined_names(forms) -> Set[str]:
    """Functions, macros, structure functions, conditions, variables and CFFI
    Lisp names a list of top-level forms defines."""
    out: Set[str] = set()

    def walk(form):
        if not isinstance(form, list) or not form:
            return
        head = form[0]
        if head in ("progn", "eval-when"):
            for f in form[1:]:
                walk(f)
            return
        if head in DEFINERS_FUNCTION or head in DEFINERS_VARIABLE or head == "define-condition":
            if len(form) > 1 and isinstance(form[1], Sym):
                out.add(str(form[1]))
            elif len(form) > 1 and isinstance(form[1], list) and form[1] and form[1][0] == "setf":
                out.add("setf " + str(form[1][1]))
        elif head == "defstruct":
            out.update(struct_names(form))
        elif head == "cffi:defcfun":
            spec = form[1]
            if isinstance(spec, list) and len(spec) > 1 and isinstance(spec[1], Sym):
                out.add(str(spec[1]))
        elif head in ("cffi:defcstruct", "cffi:define-foreign-library", "cffi:defctype"):
            if len(form) > 1:
                n = form[1][0] if isinstance(form[1], list) else form[1]
                if isinstance(n, Sym):
                    out.add(str(n))
        elif head == "feature-+" or head == "feature--":
            walk(form[1][1])

    for f in forms:
        walk(f)
    return out
