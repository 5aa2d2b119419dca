"""2-bit (ternary) weights: packed modules and the int8 projection kept 2-bit resident on the GPU."""
