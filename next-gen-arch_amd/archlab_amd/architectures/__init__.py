"""Module layout mirrors ``archlab.architectures`` for the simplicial path."""
