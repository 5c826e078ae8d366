"""Attention backends (only CCGQA)."""
