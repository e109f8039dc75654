"""Parity oracle (test infrastructure only; never imported by nanochat_amd)."""
