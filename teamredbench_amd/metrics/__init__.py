"""Built-in metric plugins."""
