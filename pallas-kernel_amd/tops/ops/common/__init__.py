"""Shared chunked-state scans (mirror of the reference's ``tops.ops.common``)."""
