"""CPU oracle of the DFlash draft forward (test infrastructure only; see dflash_oracle)."""
