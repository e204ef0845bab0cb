"""Applications built on the operator library (iron/applications)."""
