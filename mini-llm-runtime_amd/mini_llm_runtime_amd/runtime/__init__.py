"""Serving-runtime pieces on the paged attention path."""
