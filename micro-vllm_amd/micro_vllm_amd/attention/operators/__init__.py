"""Attention operators: the contract, the registry and the gfx950 backend."""
