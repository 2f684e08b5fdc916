"""The switch INTEGRATION.md documents leaves the reference's callers working unchanged (CPU, no kernel runs).

tests/golden/call_site_imports.json holds, as data, the names each reference call site imports from the
modules on the hot path, the module-level names of the reference modules this package rebinds into, and the
reference's parameter names. The tests check that:
  * with this package first on sys.path, the only reference module names it shadows are the four it replaces
    wholesale (tree_gdn_kernel, mode_attention, tree_logits, tree_build_ext), and those provide every name
    their callers import, with the reference's parameters;
  * ``ddtree_hf_ops.install()`` leaves the reference's ``ddtree`` module in place (its decode loop and switches
    still import) and points compile_ddtree_tree / follow_verified_tree / compact_dynamic_cache at this
    package, also in a module that imported one of them by name before the switch;
  * ``ddtree_sglang_ops.install()`` does the same for the SGLang patch's ``ddtree_utils`` and
    ``ddtree_mode_attention``, before or after the worker module's ``from ... import`` of them.
The reference modules are not imported: stand-ins carry their names (sentinels), so the tests show which
object each imported name resolves to after the switch.
"""

import importlib
import importlib.util
import inspect
import json
import os
import sys
import types

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "multi-future-drafting_amd")
DATA = json.load(open(os.path.join(REPO, "tests", "golden", "call_site_imports.json")))
WHOLESALE = set(DATA["hf"]["wholesale"])


class Sentinel:
    """Stands for an object of a reference module."""

    def __init__(self, module, name):
        self.where = f"{module}.{name}"

    def __repr__(self):
        return f"<reference {self.where}>"


def stand_in(name, defined):
    mod = types.ModuleType(name)
    for n in defined:
        setattr(mod, n, Sentinel(name, n))
    return mod


def from_import(module, names):
    """What ``from module import names`` binds, resolved through sys.modules as the import statement does."""
    mod = importlib.import_module(module)
    return {n: getattr(mod, n) for n in names}


def package_module_names():
    names = set()
    for entry in os.listdir(PKG):
        if entry.endswith(".py"):
            names.add(entry[:-3])
        elif os.path.isdir(os.path.join(PKG, entry)) and os.path.exists(os.path.join(PKG, entry, "__init__.py")):
            names.add(entry)
    return names


def test_package_shadows_only_the_wholesale_modules():
    reference_names = (set(DATA["hf"]["wholesale"]) | set(DATA["hf"]["kept"]) | set(DATA["sglang"]["imports"])
                       | {"ddtree_async", "ddtree_worker_v2", "dflash_info_v2", "spec_info"})
    shadowed = package_module_names() & reference_names
    assert shadowed == WHOLESALE, f"the package would shadow {sorted(shadowed - WHOLESALE)}"


def test_wholesale_modules_provide_every_imported_name(monkeypatch):
    monkeypatch.syspath_prepend(PKG)
    for module, sites in DATA["hf"]["wholesale"].items():
        spec = importlib.util.find_spec(module)
        assert spec is not None and os.path.dirname(spec.origin) == PKG, f"{module} does not resolve to the package"
        mod = importlib.import_module(module)
        for site, names in sites.items():
            missing = [n for n in names if not hasattr(mod, n)]
            assert not missing, f"{site}: {module} lacks {missing}"


def _accepts(fn, positional, keyword_only, where):
    """fn takes the reference's positional parameters in order (by position and by name) and its keyword-only
    ones by name; any further parameter of fn has a default."""
    params = list(inspect.signature(fn).parameters.values())
    if params and params[0].name == "self":
        params = params[1:]
    by_name = {p.name: p for p in params}
    pos_kinds = (inspect.Parameter.POSITIONAL_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD)
    ours_pos = [p.name for p in params if p.kind in pos_kinds]
    assert ours_pos[: len(positional)] == positional, f"{where}: positional {ours_pos} vs the reference's {positional}"
    for n in keyword_only:
        p = by_name.get(n)
        assert p is not None and p.kind in (inspect.Parameter.KEYWORD_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD), \
            f"{where}: keyword {n!r} not accepted"
    extra = [p for p in params if p.name not in positional and p.name not in keyword_only
             and p.kind not in (inspect.Parameter.VAR_POSITIONAL, inspect.Parameter.VAR_KEYWORD)]
    assert all(p.default is not inspect.Parameter.empty for p in extra), \
        f"{where}: parameters {[p.name for p in extra if p.default is inspect.Parameter.empty]} have no default"


def _ours(qualified):
    """The package object that replaces the reference's ``module.name[.method]``."""
    module, name = qualified.split(".", 1)
    owner = {"ddtree": "ddtree_hf_ops", "ddtree_utils": "ddtree_sglang_ops",
             "ddtree_mode_attention": "paged_mode_attention"}.get(module, module)
    obj = importlib.import_module(owner)
    for part in name.split("."):
        obj = getattr(obj, part)
    if inspect.isclass(obj):
        obj = obj.__init__
    return obj


def test_signatures_take_the_reference_arguments(monkeypatch):
    monkeypatch.syspath_prepend(PKG)
    for qualified, spec in DATA["signatures"].items():
        if qualified.startswith("_"):
            continue
        positional, keyword_only = spec
        _accepts(_ours(qualified), positional, keyword_only, qualified)


def test_hf_switch_keeps_the_reference_ddtree(monkeypatch):
    monkeypatch.syspath_prepend(PKG)
    ref = stand_in("ddtree", DATA["hf"]["defined"]["ddtree"])
    monkeypatch.setitem(sys.modules, "ddtree", ref)
    # a module that imported one of the functions by name before the switch
    early = types.ModuleType("early_caller")
    early.compact_dynamic_cache = ref.compact_dynamic_cache
    monkeypatch.setitem(sys.modules, "early_caller", early)
    import ddtree_hf_ops

    old = ddtree_hf_ops.install()
    rebound = DATA["hf"]["rebind"]["ddtree"]
    assert set(old) == set(rebound) and all(isinstance(o, Sentinel) for o in old.values())
    for site, names in DATA["hf"]["kept"]["ddtree"].items():
        got = from_import("ddtree", names)
        for n, obj in got.items():
            if n in rebound:
                assert obj is getattr(ddtree_hf_ops, n), f"{site}: {n} not switched"
            else:
                assert isinstance(obj, Sentinel) and obj.where == f"ddtree.{n}", f"{site}: {n} replaced"
    assert early.compact_dynamic_cache is ddtree_hf_ops.compact_dynamic_cache
    # the rest of the reference module is untouched
    for n in DATA["hf"]["defined"]["ddtree"]:
        if n not in rebound:
            assert getattr(ref, n).where == f"ddtree.{n}"


def _sglang_stand_ins(monkeypatch):
    pkg = DATA["sglang"]["package"]
    parts = pkg.split(".")
    for i in range(1, len(parts) + 1):
        name = ".".join(parts[:i])
        mod = types.ModuleType(name)
        mod.__path__ = []
        monkeypatch.setitem(sys.modules, name, mod)
        if i > 1:
            setattr(sys.modules[".".join(parts[: i - 1])], parts[i - 1], mod)
    mods = {}
    for short, defined in DATA["sglang"]["defined"].items():
        mod = stand_in(f"{pkg}.{short}", defined)
        monkeypatch.setitem(sys.modules, f"{pkg}.{short}", mod)
        setattr(sys.modules[pkg], short, mod)
        mods[short] = mod
    return pkg, mods


def _worker_imports(pkg, monkeypatch):
    """The worker module's ``from ...ddtree_utils import (...)`` and ``...ddtree_mode_attention import ...``
    (P:2003-2030), bound into a module object."""
    worker = types.ModuleType(f"{pkg}.ddtree_worker_v2")
    for short, site in (("ddtree_utils", "P:2004-2030"), ("ddtree_mode_attention", "P:2003")):
        for n, obj in from_import(f"{pkg}.{short}", DATA["sglang"]["imports"][short][site]).items():
            setattr(worker, n, obj)
    monkeypatch.setitem(sys.modules, worker.__name__, worker)
    return worker


def _check_sglang(pkg, worker):
    import ddtree_sglang_ops
    import paged_mode_attention

    ours = {"ddtree_utils": ddtree_sglang_ops, "ddtree_mode_attention": paged_mode_attention}
    for short, sites in DATA["sglang"]["imports"].items():
        rebound = DATA["sglang"]["rebind"][short]
        for site, names in sites.items():
            for n, obj in from_import(f"{pkg}.{short}", names).items():
                if n in rebound:
                    assert obj is getattr(ours[short], n), f"{site}: {n} not switched"
                else:
                    assert isinstance(obj, Sentinel) and obj.where == f"{pkg}.{short}.{n}", f"{site}: {n} replaced"
    for n in DATA["sglang"]["imports"]["ddtree_utils"]["P:2004-2030"]:
        want = getattr(ddtree_sglang_ops, n) if n in DATA["sglang"]["rebind"]["ddtree_utils"] else None
        if want is not None:
            assert getattr(worker, n) is want, f"worker's {n} not switched"
        else:
            assert isinstance(getattr(worker, n), Sentinel)
    assert worker.PagedModeAttention is paged_mode_attention.PagedModeAttention


def test_sglang_switch_after_the_worker_import(monkeypatch):
    monkeypatch.syspath_prepend(PKG)
    pkg, mods = _sglang_stand_ins(monkeypatch)
    worker = _worker_imports(pkg, monkeypatch)
    import ddtree_sglang_ops

    old = ddtree_sglang_ops.install()
    assert old["build_trees"] is None  # the device builder is added, the patch has no such name
    assert all(isinstance(old[n], Sentinel) for n in DATA["sglang"]["rebind"]["ddtree_utils"])
    _check_sglang(pkg, worker)
    assert isinstance(mods["ddtree_utils"]._CPP_SOURCE, Sentinel)  # ddtree_async still compiles its own source


def test_sglang_switch_before_the_worker_import(monkeypatch):
    monkeypatch.syspath_prepend(PKG)
    pkg, _ = _sglang_stand_ins(monkeypatch)
    import ddtree_sglang_ops

    ddtree_sglang_ops.install()
    worker = _worker_imports(pkg, monkeypatch)
    _check_sglang(pkg, worker)
