"""patch(model, rules): route a model's Linear layers and attention cores through Schemes
(mxq/nn/_patch.py:1-287).

    rules = [("lm_head", None),            # selector, value; a selector is a name pattern (fnmatch, * wildcard),
             ("*.mlp.down_proj", FP6),     #   a module type, or a callable (name, module, parent) -> bool
             (is_attention, None),         # value None: keep the layer as it is
             (nn.Linear, FP8)]             # value Scheme: the Linear becomes an MXLinear through it
    handle = patch(model, rules)           # the first rule that matches a layer decides it
    print(handle); handle.revert()
    patch(model, rules, dry_run=True)      # print what would happen, change nothing

A value (qk, pv) -- two Schemes -- makes the rule choose attention modules (a module holding q_proj and k_proj)
instead of Linears; their core then runs through mxq.nn.attend under the "mxq" transformers attention
implementation, and attention modules no such rule chose keep sdpa.  vector= sets the precision of softmax and
RMSNorm steps (mxq.nn._vector): softmax sends every attention module through attend (the EXACT core where no
rule chose one); rmsnorm replaces the forward of every module whose class name ends in RMSNorm, after checking
that the replacement reproduces it bit for bit.

Checks, all before the model is touched: every rule must choose something; one layer reachable under several
names (a module held twice) must get one answer; every Scheme runs once on a tiny matmul, on the device of the
model's parameters.
"""
from dataclasses import dataclass, field
from fnmatch import fnmatchcase
from functools import partial
from typing import Callable, Dict, List, Optional, Sequence, Tuple, Union

import torch
from torch import nn

from ..scheme import Scheme
from ._attention import NAME as _CORE_NAME, attend, register
from ._linear import MXLinear
from ._vector import EXACT, resolve, rmsnorm

__all__ = ["patch", "is_attention"]

Selector = Union[str, type, Callable[[str, nn.Module, nn.Module], bool]]
Rule = Tuple[Selector, Union[None, Scheme, Tuple[Scheme, Scheme]]]


def is_attention(name: str, module: nn.Module, parent: nn.Module) -> bool:
    """A Linear whose parent holds q_proj and k_proj: an attention projection (MXQuant's eval_complete.py test,
    mxq/nn/_patch.py:123-131)."""
    return _is_attention_module(parent)


def _is_attention_module(module: nn.Module) -> bool:
    return hasattr(module, "q_proj") and hasattr(module, "k_proj")


def _is_core_value(value) -> bool:
    return isinstance(value, tuple) and len(value) == 2 and all(isinstance(s, Scheme) for s in value)


def _selects(selector: Selector, name: str, module: nn.Module, parent: nn.Module) -> bool:
    if isinstance(selector, str):
        return fnmatchcase(name, selector)
    if isinstance(selector, type):
        return isinstance(module, selector)
    return bool(selector(name, module, parent))


@dataclass
class _Site:
    """One place a module runs from: an attribute of a parent (Linear) or a module object (attention).
    `names` are every name the model reaches it under, `hits` the first matching rule of each."""
    module: nn.Module
    parent: Optional[nn.Module]
    names: List[str] = field(default_factory=list)
    hits: List[Optional[int]] = field(default_factory=list)

    @property
    def rule(self) -> Optional[int]:
        return self.hits[0]


def _collect(model: nn.Module, rules: Sequence[Rule], kind: str) -> Dict[tuple, _Site]:
    """Walk every name (duplicates included) and record the first matching rule of `kind` per name."""
    by_name = dict(model.named_modules(remove_duplicate=False))
    wanted = [i for i, (_, value) in enumerate(rules) if _is_core_value(value) == (kind == "core")]
    sites: Dict[tuple, _Site] = {}
    for name, module in model.named_modules(remove_duplicate=False):
        if not name:
            continue
        if kind == "linear" and not isinstance(module, nn.Linear):
            continue
        if kind == "core" and not _is_attention_module(module):
            continue
        parent_name, _, leaf = name.rpartition(".")
        parent = by_name[parent_name]
        hit = next((i for i in wanted if _selects(rules[i][0], name, module, parent)), None)
        key = (id(parent), leaf) if kind == "linear" else (id(module),)
        site = sites.setdefault(key, _Site(module, parent))
        site.names.append(name)
        site.hits.append(hit)
    used = {h for s in sites.values() for h in s.hits}
    unused = [i for i in wanted if i not in used]
    if unused and kind == "linear":
        raise ValueError(f"rules {unused} choose no Linear layer (misspelt, or hidden behind an earlier rule): "
                         f"{[rules[i][0] for i in unused]}")
    if unused:
        raise ValueError(f"rules {unused} choose no attention module (one holding q_proj and k_proj): "
                         f"{[rules[i][0] for i in unused]}")
    return sites


def _require_agreement(sites: Dict[tuple, _Site], kind: str) -> None:
    for site in sites.values():
        if len(set(site.hits)) < 2:
            continue
        if kind == "core":
            raise ValueError(f"{site.names} are the same attention module but match different rules; "
                             "one of them has to go")
        raise ValueError(f"{site.names} are the same layer but match different rules {site.hits}; "
                         "one of them has to go")


def _param_device(model: nn.Module) -> torch.device:
    p = next(model.parameters(), None)
    return p.device if p is not None else torch.device("cpu")


def _try_scheme(scheme: Scheme, device: torch.device) -> None:
    """One seeded matmul over three blocks of K and two `rows` groups of columns."""
    gen = torch.Generator().manual_seed(0)
    K, n = 3 * scheme.block_size, 2 * scheme.rows
    A, B = torch.randn(K, n, generator=gen), torch.randn(K, n, generator=gen)
    scheme.matmul(A.to(device), B.to(device))


def _try_core(qk: Scheme, pv: Scheme, device: torch.device) -> None:
    """attend on one KV head shared by two query heads, over whole key blocks and whole `rows` groups."""
    gen = torch.Generator().manual_seed(0)
    T = 2 * max(qk.block_size, pv.block_size) * max(qk.rows, pv.rows)
    q, k, v = (torch.randn(1, heads, T, 32, generator=gen).to(device) for heads in (2, 1, 1))
    attend(q, k, v, None, 32 ** -0.5, qk, pv)


def _epsilon(module: nn.Module) -> float:
    for attr in ("variance_epsilon", "eps"):
        value = getattr(module, attr, None)
        if isinstance(value, float):
            return value
    raise ValueError(f"{type(module).__name__}: no float variance_epsilon or eps attribute")


def _verify_rmsnorm(name: str, module: nn.Module) -> float:
    """The unrounded replacement must equal the module's own output bit for bit; returns the module's eps."""
    weight = getattr(module, "weight", None)
    if not isinstance(weight, torch.Tensor) or weight.ndim != 1:
        raise ValueError(f"{name} ({type(module).__name__}): no 1-D weight, not the RMSNorm mxq knows")
    eps = _epsilon(module)
    gen = torch.Generator().manual_seed(0)
    x = (3 * torch.randn(3, weight.shape[0], generator=gen)).to(device=weight.device, dtype=weight.dtype)
    with torch.no_grad():
        expect, got = module(x), rmsnorm(x, weight, eps, None)
    if expect.dtype != got.dtype or not torch.equal(expect, got):
        raise ValueError(f"{name} ({type(module).__name__}) does not compute weight · x / sqrt(mean(x²) + eps) the way "
                         "transformers' LlamaRMSNorm does; vector rmsnorm cannot replace it")
    return eps


def _norm_forward(module: nn.Module, eps: float, precision: Optional[str], x: torch.Tensor) -> torch.Tensor:
    return rmsnorm(x, module.weight, eps, precision)


def _set_implementation(model: nn.Module, name: str) -> None:
    if hasattr(model, "set_attn_implementation"):
        model.set_attn_implementation(name)
    else:
        model.config._attn_implementation = name


def _strip_core(module: nn.Module) -> None:
    for attr in ("_mxq_core", "_mxq_vector"):
        if hasattr(module, attr):
            delattr(module, attr)


def _strip_forward(module: nn.Module) -> None:
    del module.forward                                                             # the class's forward again


class Handle:
    """The result of patch.

    table: one row per Linear name -- (name, in_features, out_features, rule index or None, Scheme name or None)
    cores: one row per attention-module name -- (name, rule index or None, (qk name, pv name) or None = sdpa)
    vector: the resolved {op: precision}; norms: the RMSNorm module names whose forward was replaced
    revert(): undo every change, last first."""

    def __init__(self, table, cores, vector, norms):
        self.table, self.cores, self.vector, self.norms = table, cores, vector, norms
        self._undo: List[Callable[[], None]] = []

    def revert(self) -> None:
        while self._undo:
            self._undo.pop()()

    def __str__(self) -> str:
        w = max([5] + [len(r[0]) for r in self.table] + [len(r[0]) for r in self.cores])
        out = [f"{'layer':<{w}}  {'in':>6} {'out':>6}  rule  scheme"]
        for name, k, n, rule, scheme in self.table:
            what = "no rule" if rule is None else (scheme or "left as is")
            out.append(f"{name:<{w}}  {k:>6} {n:>6}  {'-' if rule is None else rule:>4}  {what}")
        if any(names is not None for _, _, names in self.cores):
            out.append(f"{'attention core':<{w}}  {'':13}  rule  Q·Kᵀ, P·V")
            for name, rule, names in self.cores:
                what = "sdpa (no rule)" if names is None else ", ".join(names)
                if rule is None and names is not None:
                    what += "  (vector softmax)"
                out.append(f"{name:<{w}}  {'':13}  {'-' if rule is None else rule:>4}  {what}")
        if any(self.vector.values()):
            count = {"softmax": sum(names is not None for _, _, names in self.cores), "rmsnorm": len(self.norms)}
            parts = [f"{op} {p} ({count[op]} modules)" if p else f"{op} as transformers"
                     for op, p in self.vector.items()]
            out.append("vector  " + ", ".join(parts))
        return "\n".join(out)


def patch(model: nn.Module, rules: Sequence[Rule], chunk: Optional[int] = None, dry_run: bool = False,
          cache_weights: bool = True, vector=None) -> Handle:
    """Apply `rules` to `model` (see the module docstring); chunk and cache_weights go to every MXLinear."""
    vector = resolve(vector)
    for i, rule in enumerate(rules):
        if len(rule) != 2 or not (rule[1] is None or isinstance(rule[1], Scheme) or _is_core_value(rule[1])):
            raise ValueError(f"rule {i} must be (selector, Scheme or None or (qk Scheme, pv Scheme)), got {rule!r}")

    linears = _collect(model, rules, "linear")
    cores = _collect(model, rules, "core")
    _require_agreement(cores, "core")
    _require_agreement(linears, "linear")

    if vector["softmax"] and not cores:
        raise ValueError("vector softmax: the model has no attention module (one holding q_proj and k_proj)")
    norms: Dict[int, Tuple[str, nn.Module]] = {}
    if vector["rmsnorm"]:
        for name, module in model.named_modules(remove_duplicate=False):
            if name and type(module).__name__.endswith("RMSNorm"):
                norms.setdefault(id(module), (name, module))
        if not norms:
            raise ValueError("vector rmsnorm: the model has no module whose class name ends in RMSNorm")

    def core_for(rule: Optional[int]):
        if rule is not None:
            return rules[rule][1]
        return (EXACT, EXACT) if vector["softmax"] else None

    device = _param_device(model)                                                  # fail now, not mid-run
    for _, value in rules:
        if isinstance(value, Scheme):
            _try_scheme(value, device)
    for _, value in rules:
        if _is_core_value(value):
            _try_core(*value, device)
    if vector["softmax"] and any(site.rule is None for site in cores.values()):
        _try_core(EXACT, EXACT, device)
    eps = {key: _verify_rmsnorm(name, module) for key, (name, module) in norms.items()}

    order = {name: i for i, (name, _) in enumerate(model.named_modules(remove_duplicate=False))}
    table = sorted(((name, site.module.in_features, site.module.out_features, hit,
                     rules[hit][1].name if hit is not None and isinstance(rules[hit][1], Scheme) else None)
                    for site in linears.values() for name, hit in zip(site.names, site.hits)),
                   key=lambda row: order[row[0]])
    core_rows = sorted(((name, site.rule, None if core_for(site.rule) is None
                         else tuple(s.name for s in core_for(site.rule)))
                        for site in cores.values() for name in site.names), key=lambda row: order[row[0]])
    handle = Handle(table, core_rows, vector, [name for name, _ in norms.values()])
    if dry_run:
        print(handle)
        return handle

    for site in linears.values():
        value = None if site.rule is None else rules[site.rule][1]
        if value is None:
            continue
        leaf = site.names[0].rpartition(".")[2]
        setattr(site.parent, leaf, MXLinear(site.module, value, chunk, cache_weights))
        handle._undo.append(partial(setattr, site.parent, leaf, site.module))

    routed = [(site.module, core_for(site.rule)) for site in cores.values() if core_for(site.rule) is not None]
    if routed:
        register()
        before = model.config._attn_implementation
        for module, core in routed:
            module._mxq_core = core
            if vector["softmax"]:
                module._mxq_vector = vector["softmax"]
            handle._undo.append(partial(_strip_core, module))
        _set_implementation(model, _CORE_NAME)
        handle._undo.append(partial(_set_implementation, model, before))

    for key, (_, module) in norms.items():
        module.forward = partial(_norm_forward, module, eps[key], vector["rmsnorm"])
        handle._undo.append(partial(_strip_forward, module))
    return handle
