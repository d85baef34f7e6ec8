"""CPU oracle of the block-sparse GEMM path — test infrastructure only (see bsg_oracle.py)."""
