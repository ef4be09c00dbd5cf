"""Argument errors of the operators (raised before any kernel launch)."""


class ArgumentError(ValueError, AssertionError):
    """Invalid operator argument.  The reference checks its arguments with ``assert``
    (``src/flag_attn/paged.py:45-46``, ``split_kv.py:282-289``), so this is an
    ``AssertionError`` as well as a ``ValueError``."""
