"""CPU oracle for MatMulNBits — test infrastructure only (see matmul_nbits.py)."""
