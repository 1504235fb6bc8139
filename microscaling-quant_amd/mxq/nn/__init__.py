"""mxq.nn -- Schemes inside a model (mxq/nn/__init__.py:1-17).

    MXLinear(linear, scheme)     one nn.Linear computed through one Scheme (inference only)
    patch(model, rules)          a Scheme per layer name or type, first matching rule wins; (qk, pv) for a core
    is_attention                 selector for the attention projections
    attend(q, k, v, mask, scale, qk, pv)   the attention core with Q K^T and P V through two Schemes
"""
from ._attention import attend
from ._linear import MXLinear
from ._patch import is_attention, patch

__all__ = ["MXLinear", "patch", "is_attention", "attend"]
