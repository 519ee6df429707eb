"""Operator packages (``tops.ops.gla``)."""
