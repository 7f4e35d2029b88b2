"""Drop-in variant modules (reference variant contract: META, prepare, run, dequant, ...)."""
