"""fa2: FlashAttention-2 forward for AMD MI355X (gfx950). The entry point is fa2.kernel.attention."""
