"""Public constants.

SUPPORTED_K extends the reference's (4, 8, 16) (torchbvh/_constants.py:1) with
32, which the ragged k=32 workload needs; every other k is still rejected.
"""

SUPPORTED_K = (4, 8, 16, 32)
SUPPORTED_DIMS = (2, 3)
# Squared distance at or below which a neighbour counts as an exact hit in
# the displaced-query interpolation (torchbvh/_constants.py:3).
EXACT_DISTANCE_EPSILON = 1.0e-12
