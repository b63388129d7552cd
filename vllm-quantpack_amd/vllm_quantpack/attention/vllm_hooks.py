"""How this package attaches itself to a running vLLM.

vLLM finds the int4 attention through names it looks up at call time: module globals of its int4 ops module, methods
of the Triton backend and its metadata builder, and the KV-cache dtype registry. Each attachment here is a `Hook`:
one attribute of one vLLM object and the value to put there. A `HookSet` applies hooks, keeps every replaced value
next to the object it came from, and can put them back, so that

* applying the same hooks twice changes nothing (a replacement carries the marker `_quantpack`);
* a test, or a process that turns the package off again, can restore vLLM exactly (`HookSet.restore`);
* `HookSet.applied` lists what was installed, for the log line and for tests.

The vLLM attribute names used by the hooks are vLLM's interface (the reference plugin attaches to the same ones,
k8v4_kv.py:89-166 and int4_kv.py:229-257); everything else here is this package's own.
"""
from __future__ import annotations

import contextlib
import importlib
from dataclasses import dataclass
from typing import Any, Callable

MARK = "_quantpack"
_MISSING = object()


def marked(fn: Any) -> bool:
    """Whether `fn` (a function, a classmethod object or a bound method) is one of this package's replacements."""
    fn = getattr(fn, "__func__", fn)
    return bool(getattr(fn, MARK, False))


def mark(fn: Callable) -> Callable:
    setattr(fn, MARK, True)
    return fn


@dataclass
class Hook:
    owner: Any            # a module or a class
    name: str
    value: Any            # the replacement (functions are marked when applied)
    what: str = ""        # one line for the log


class HookSet:
    def __init__(self):
        self._saved: list[tuple[Any, str, Any]] = []
        self.applied: list[str] = []

    def apply(self, hook: Hook) -> bool:
        """Install one hook; False when the owner already holds one of this package's replacements there."""
        current = (hook.owner.__dict__.get(hook.name, _MISSING) if isinstance(hook.owner, type)
                   else getattr(hook.owner, hook.name, _MISSING))
        if current is not _MISSING and marked(current):
            return False
        fn = getattr(hook.value, "__func__", hook.value)
        if callable(fn):
            mark(fn)
        elif current is not _MISSING and current == hook.value:
            return False        # a plain value already in place
        self._saved.append((hook.owner, hook.name, current))
        setattr(hook.owner, hook.name, hook.value)
        self.applied.append(hook.what or f"{getattr(hook.owner, '__name__', hook.owner)}.{hook.name}")
        return True

    def restore(self) -> None:
        """Put every replaced attribute back (attributes that did not exist are removed), newest first."""
        while self._saved:
            owner, name, old = self._saved.pop()
            if old is _MISSING:
                with contextlib.suppress(AttributeError):
                    delattr(owner, name)
            else:
                setattr(owner, name, old)
        self.applied.clear()


HOOKS = HookSet()   # the hooks of this process


def find(path: str, *attrs: str):
    """The module at `path` and the named attributes of it (dotted names allowed), or raise what the import raises:
    the caller turns a vLLM without the feature into "left stock"."""
    mod = importlib.import_module(path)
    out = [mod]
    for a in attrs:
        obj = mod
        for part in a.split("."):
            obj = getattr(obj, part)
        out.append(obj)
    return out


@contextlib.contextmanager
def module_value(module, name: str, value):
    """Give a module global another value for the duration of a block (for code that reads it as a constant)."""
    old = getattr(module, name)
    setattr(module, name, value)
    try:
        yield
    finally:
        setattr(module, name, old)
