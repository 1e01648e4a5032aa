"""Execution providers for dispatch winners."""
