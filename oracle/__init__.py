"""CPU oracle of the TileOPs forward-operator path -- test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg,
never by the tileops package.  See tileops_oracle.py.
"""

from oracle import tileops_oracle

__all__ = ["tileops_oracle"]
