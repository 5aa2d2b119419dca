"""1-bit (sign) weights: export codes, the gfx950 native layout, the Int8MmaLayer operators and the provider seam."""
