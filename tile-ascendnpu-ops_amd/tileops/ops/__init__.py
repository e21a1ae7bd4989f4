"""Operator classes.  Import the families you use, e.g.
``from tileops.ops.elementwise import HardswishFwdOp``; this module stays
light so that importing one family does not load the others."""

from tileops.ops.op_base import Op

__all__ = ["Op"]
