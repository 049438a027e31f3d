"""Serving-runtime structures around the paged-KV path."""
