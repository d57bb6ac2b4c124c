"""The Lisp INTEGRATION.md asks a maintainer to add to llambda calls only
functions and macros that exist: those its own blocks define, the
reference's (tests/golden/reference_symbols.json, written from the
reference's sources by tests/golden/make_reference_symbols.py), Common Lisp's
and the libraries llambda already loads (CFFI, UIOP, SBCL's sb-thread).
CPU only; nothing is evaluated."""
import json
import os
import re

import pytest

from lisp_forms import Sym, defined_names, read_all

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

# Common Lisp operators the blocks use (every one is an external symbol of
# the COMMON-LISP package, CLHS 1.9).
COMMON_LISP = {
    "and", "acons", "assoc", "char-code", "coerce", "concatenate", "cond", "declare", "defconstant",
    "defstruct", "defun", "defvar", "define-condition", "dolist", "dotimes", "ensure-directories-exist",
    "error", "etypecase", "eq", "flet", "format", "funcall", "gethash", "getf", "if", "ignore",
    "in-package", "lambda", "ldb", "byte", "length", "let", "let*", "loop", "macrolet", "make-hash-table",
    "map", "mapcar", "merge-pathnames", "min", "multiple-value-bind", "not", "null", "or", "progn",
    "push", "pushnew", "remhash", "remove", "search", "setf", "string=", "subseq", "typep", "unless",
    "unwind-protect", "values", "when", "with-open-file", "write-byte", "zerop", "+", "-", "*",
    "=", "<", ">", "1+", "1-", "apply", "list", "car", "cdr", "function", "quote", "the",
    "nil", "t", "defmacro", "handler-case", "typecase", "case", "ecase", "block", "return-from",
}
# operators of the libraries llambda.asd already depends on (llambda.asd:6) and UIOP
LIBRARY_PACKAGES = ("cffi:", "sb-thread:", "uiop:", "sb-ext:")

# special forms and macros whose arguments are not all evaluated forms
_BINDING_BODY = {"let", "let*"}


def lisp_blocks(text):
    return re.findall(r"```lisp\n(.*?)```", text, flags=re.S)


class Walker:
    """Collect (name, context) for every operator a form calls, skipping
    lambda lists, binding names, quoted data and declarations."""

    def __init__(self):
        self.calls = []

    def forms(self, forms, ctx):
        for f in forms:
            self.form(f, ctx)

    def form(self, f, ctx, local=frozenset()):
        if isinstance(f, list):
            if not f:
                return
            head = f[0]
            if isinstance(head, list):
                if head and head[0] == "lambda":
                    self.form(head, ctx, local)
                    self.forms_local(f[1:], ctx, local)
                    return
                raise AssertionError(f"{ctx}: a list in operator position: {head!r}")
            if not isinstance(head, Sym):
                return
            self.special(head, f, ctx, local)

    def forms_local(self, forms, ctx, local):
        for x in forms:
            self.form(x, ctx, local)

    def call(self, name, ctx, local):
        if name not in local:
            self.calls.append((str(name), ctx))

    def body(self, forms, ctx, local):
        for x in forms:
            if isinstance(x, list) and x and x[0] == "declare":
                continue
            self.form(x, ctx, local)

    def special(self, head, f, ctx, local):  # noqa: C901 - one case per form
        h = str(head)
        if h in ("quote", "quasiquote", "read-eval", "vector", "in-package", "declare",
                 "define-condition", "defstruct", "cffi:defcfun", "cffi:defcstruct",
                 "cffi:define-foreign-library", "defconstant"):
            return
        if h == "function":
            target = f[1]
            if isinstance(target, Sym):
                self.call(target, ctx, local)
            else:
                self.form(target, ctx, local)
            return
        if h in ("defun", "defmacro"):
            self.body(f[3:], f"{ctx}/{f[1]}", local)
            return
        if h in ("defvar", "defparameter"):
            if len(f) > 2:
                self.form(f[2], ctx, local)
            return
        if h == "lambda":
            self.body(f[2:], ctx, local)
            return
        if h in _BINDING_BODY:
            for b in f[1]:
                if isinstance(b, list) and len(b) > 1:
                    self.form(b[1], ctx, local)
            self.body(f[2:], ctx, local)
            return
        if h in ("flet", "labels", "macrolet"):
            names = {str(d[0]) for d in f[1]}
            inner = local | names
            for d in f[1]:
                if h != "macrolet":  # a macrolet body is a template
                    self.body(d[2:], ctx, inner if h == "labels" else local)
            self.body(f[2:], ctx, inner)
            return
        if h == "multiple-value-bind":
            self.form(f[2], ctx, local)
            self.body(f[3:], ctx, local)
            return
        if h in ("dotimes", "dolist"):
            self.form(f[1][1], ctx, local)
            self.body(f[2:], ctx, local)
            return
        if h in ("cffi:with-foreign-object", "cffi:with-foreign-objects"):
            specs = [f[1]] if h == "cffi:with-foreign-object" else f[1]
            for s in specs:
                for x in s[2:]:  # count forms
                    self.form(x, ctx, local)
                self.form(s[1], ctx, local)  # the type, evaluated by the macro
            self.body(f[2:], ctx, local)
            return
        if h == "cffi:with-pointer-to-vector-data":
            self.form(f[1][1], ctx, local)
            self.body(f[2:], ctx, local)
            return
        if h == "sb-thread:with-mutex":
            self.form(f[1][0], ctx, local)
            self.body(f[2:], ctx, local)
            return
        if h == "with-open-file":
            for x in f[1][1:]:
                self.form(x, ctx, local)
            self.body(f[2:], ctx, local)
            return
        if h in ("etypecase", "typecase", "case", "ecase"):
            self.call(head, ctx, local)
            self.form(f[1], ctx, local)
            for clause in f[2:]:
                self.body(clause[1:], ctx, local)
            return
        if h == "handler-case":
            self.call(head, ctx, local)
            self.form(f[1], ctx, local)
            for clause in f[2:]:
                self.body(clause[2:], ctx, local)
            return
        if h == "cond":
            for clause in f[1:]:
                self.body(clause, ctx, local)
            return
        if h == "loop":
            self.call(head, ctx, local)
            items = f[1:]
            i = 0
            while i < len(items):
                x = items[i]
                if isinstance(x, Sym) and x in ("for", "as", "with"):
                    i += 2  # the variable or destructuring pattern
                    continue
                self.form(x, ctx, local)
                i += 1
            return
        self.call(head, ctx, local)
        for x in f[1:]:
            self.form(x, ctx, local)


@pytest.fixture(scope="module")
def integration_blocks():
    with open(os.path.join(ROOT, "INTEGRATION.md"), encoding="utf-8") as f:
        blocks = lisp_blocks(f.read())
    assert len(blocks) >= 4
    return [read_all(b) for b in blocks]


@pytest.fixture(scope="module")
def reference_names():
    with open(os.path.join(HERE, "golden", "reference_symbols.json")) as f:
        data = json.load(f)
    assert "llambda.lisp" in data["sources"]
    return set(data["names"])


def test_reference_symbol_list_covers_the_store(reference_names):
    # names the MoE hook leans on, and one it must not: the reference has no
    # with-model-runtime-lock (its idiom is sb-thread:with-mutex on
    # gguf-model-runtime-mutex, llambda.lisp:2704, 2752)
    for name in ("gguf-model-runtime-mutex", "defer-or-collect-accelerator-projections",
                 "close-retired-accelerator-projections", "make-accelerator-projection",
                 "accelerator-projection-run-mutex", "call-with-accelerator-runtime-fallback",
                 "call-with-accelerator-setup-fallback", "ensure-model-open",
                 "signal-accelerator-backend-error", "gguf-kv-value-or-nil"):
        assert name in reference_names, name
    assert "with-model-runtime-lock" not in reference_names


def test_every_called_name_is_defined(integration_blocks, reference_names):
    own = set()
    for forms in integration_blocks:
        own |= defined_names(forms)
    known = own | reference_names | COMMON_LISP
    missing, seen = [], set()
    for i, forms in enumerate(integration_blocks):
        w = Walker()
        w.forms(forms, f"block {i + 1}")
        for name, ctx in w.calls:
            seen.add(name)
            if name in known or name.startswith(LIBRARY_PACKAGES) or name.startswith(":"):
                continue
            missing.append(f"{ctx}: {name}")
    assert not missing, "undefined operators in INTEGRATION.md's Lisp:\n" + "\n".join(missing)
    # the walk reached the store calls the hook depends on
    assert {"gguf-model-runtime-mutex", "defer-or-collect-accelerator-projections",
            "call-with-accelerator-runtime-fallback", "%hip-moe-session-run",
            "check-hip-moe-status"} <= seen


def test_the_walker_finds_an_undefined_operator(reference_names):
    forms = read_all("(defun f (model) (with-model-runtime-lock (model) (g model)))"
                     "(defun g (m) (let ((x (car m))) (flet ((h (y) y)) (h x))))")
    w = Walker()
    w.forms(forms, "t")
    names = {n for n, _ in w.calls}
    assert "with-model-runtime-lock" in names and "h" not in names and "x" not in names
    assert "with-model-runtime-lock" not in reference_names | COMMON_LISP | defined_names(forms)


def test_moe_hook_changes_the_table_under_the_runtime_mutex(integration_blocks):
    """register/unregister/clear of the MoE table take the model's runtime
    mutex, and unregister/clear hand their victims to
    defer-or-collect-accelerator-projections inside it (llambda.lisp:2752-2787)."""
    defs = {}
    for forms in integration_blocks:
        for f in forms:
            if isinstance(f, list) and f and f[0] == "defun":
                defs[str(f[1])] = f

    def find(form, pred, inside=False, under_mutex=False):
        hits = []
        if isinstance(form, list) and form:
            mutex = (form[0] == "sb-thread:with-mutex" and isinstance(form[1], list)
                     and isinstance(form[1][0], list) and form[1][0][0] == "gguf-model-runtime-mutex")
            if pred(form):
                hits.append(under_mutex)
            for x in form[1:]:
                hits += find(x, pred, inside, under_mutex or mutex)
        return hits

    def calls(name):
        return lambda f: isinstance(f[0], Sym) and f[0] == name

    for name in ("register-model-hip-moe-layer", "unregister-model-hip-moe-layer",
                 "clear-model-hip-moe-layers"):
        table_writes = find(defs[name], lambda f: f[0] == "setf" and any(
            isinstance(x, list) and x and x[0] == "gethash" and "*hip-moe-layers*" in x
            for x in f[1:]) or f[0] == "remhash")
        assert table_writes and all(table_writes), name
    for name in ("unregister-model-hip-moe-layer", "clear-model-hip-moe-layers"):
        deferred = find(defs[name], calls("defer-or-collect-accelerator-projections"))
        closed = find(defs[name], calls("close-retired-accelerator-projections"))
        assert deferred and all(deferred), name
        assert closed and not any(closed), name  # closed after the lock is released
