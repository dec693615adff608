"""Attention metadata context."""
