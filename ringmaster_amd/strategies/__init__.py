"""Recurrent state passing (context-parallel linear scan)."""
