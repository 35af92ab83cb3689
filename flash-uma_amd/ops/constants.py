"""Layout constants of the rotated-frame m-blocks and the Wigner scalars (ops/constants.py:7-35).

Wigner (E, 34): row-major L=1 3x3 block at 0..8, row-major L=2 5x5 block at 9..33.
Block widths in units of C: X (gather output) 6/8/4, Y (conv1 output) 5/4/2,
Z (gate output and conv2 in/out) 3/4/2.
"""
N_WIGNER = 34
L1_OFFSET = 0
L2_OFFSET = 9

X_M0_MULT, X_M1_MULT, X_M2_MULT = 6, 8, 4
Y_M0_MULT, Y_M1_MULT, Y_M2_MULT = 5, 4, 2
Z_M0_MULT, Z_M1_MULT, Z_M2_MULT = 3, 4, 2
RAD_MULT = 12          # radial blocks per layer (6 * lmax)
INIT_RAD_MULT = 3      # radial blocks of the edge-degree embedding (lmax + 1)
EDGE_DEGREE_RESCALE = 5.0
LN_EPS = 1e-7          # ops/ln_silu.py:180

# Names of the reference's constants module (ops/constants.py:7-35).  W<r><c> is the offset of
# entry (r, c) of the per-edge Wigner scalars: rows and columns 1-3 index the L = 1 block,
# 4-8 the L = 2 block.
for _r in range(1, 4):
    for _c in range(1, 4):
        globals()[f"W{_r}{_c}"] = L1_OFFSET + 3 * (_r - 1) + (_c - 1)
for _r in range(4, 9):
    for _c in range(4, 9):
        globals()[f"W{_r}{_c}"] = L2_OFFSET + 5 * (_r - 4) + (_c - 4)
del _r, _c
S3 = 2.0 * 3.0 ** 0.5      # multiples of sqrt(3) used by the L = 2 Wigner polynomials
S3X2 = 2.0 * S3
S3X3 = 3.0 * S3
S3X4 = 4.0 * S3
TRUNC_Y_M0_MULT = Y_M0_MULT
TRUNC_Z_M0_MULT = Z_M0_MULT
