"""CPU parity oracle (test infrastructure only; see refcpu.h)."""
