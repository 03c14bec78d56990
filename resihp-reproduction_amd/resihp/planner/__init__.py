"""Pure (torch-free) pipeline schedule definitions."""
