"""Parity oracle for the GPTQ+ hot path: test infrastructure only (never the product path)."""
