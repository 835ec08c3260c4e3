"""CPU oracle of phoenix-lai's MoE FFN path: test infrastructure only (see oracle.h)."""
