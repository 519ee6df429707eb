"""Operator packages (``tops.ops.gla``, ``tops.ops.simple_gla``, ``tops.ops.common``)."""
