"""CPU oracle for the ez-ops decode hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may
import this package, and only as the checker.  The product path (the ezops
package and libezops_hip.so) never calls it.
"""

from .ops import *  # noqa: F401,F403
