"""See the package docstring of bitexact."""
