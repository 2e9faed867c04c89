"""Algorithmic work of one preconditioner update + apply (the FLOP count that the measurement divides by).

Per m x n parameter with dense factors on both sides, P = Q^T Q kept as state (the decomposition of
psgd_pro_fast.py:156-192, psgd_pro.py:107-135 for the arithmetic):
  two P1 G P2 applies (update and apply)        4 (m^2 n + m n^2)
  term1 SYRKs (upper triangle)                  m(m+1) n + n(n+1) m
  term1 Q                                       2 (m^3 + n^3)
  Procrustes products (step2; r2: 3 d^3)        4 (m^3 + n^3)
  P refresh (SYRK)                              m^2 (m+1) + n^2 (n+1)
  two norm lower bounds                         514 (m^2 + n^2)  (4 V A products of 2 * 32 flops per stored
                                                element plus one row-norm pass)
A diagonal side contributes m n per apply and nothing else.
"""
from .kron import _is_dense as is_dense  # the factor rule of psgd_pro.py:189

__all__ = ["flops_2d", "is_dense"]


def flops_2d(m, n, dense1=True, dense2=True, r2=False):
    f = 0
    f += 2 * ((2 * m * m * n if dense1 else m * n) + (2 * m * n * n if dense2 else m * n))
    for d, o, dense in ((m, n, dense1), (n, m, dense2)):
        if not dense:
            continue
        f += d * (d + 1) * o + 2 * d ** 3 + (3 if r2 else 4) * d ** 3 + d * d * (d + 1) + 514 * d * d
    return f
