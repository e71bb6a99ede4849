"""CPU oracle of the FlashAttention-2 forward (test infrastructure; see oracle/reference.py)."""
