"""Import path ``attention.attention`` / ``attention.triton_atopn`` of the reference.

Callers written against the reference (``from attention.attention import ...``,
``import attention.attention as _attn_module``) get the MI355X modules of
saga_amd.attention.  The submodules are registered under both names so that a
module global assigned through one name (``EXEMPT_LAYERS``,
``AMORTIZED_THRESHOLD_TENSOR``) is seen through the other.
"""
import sys

from saga_amd.attention import attention, triton_atopn

sys.modules[__name__ + ".attention"] = attention
sys.modules[__name__ + ".triton_atopn"] = triton_atopn
