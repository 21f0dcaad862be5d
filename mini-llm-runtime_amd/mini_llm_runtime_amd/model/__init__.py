"""Model code that calls the paged attention path."""
