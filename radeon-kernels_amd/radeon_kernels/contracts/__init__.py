"""Operator contracts (JSON resources)."""
