"""Golden vectors of the real-quant MoE path (data + the script that writes them)."""
