"""Exception type shared by the binding and the public module."""


class QuantizationError(ValueError):
    """Raised on invalid weight, scale, or group-size inputs.

    Same type and base class as Kshipra's ``engine/quantization.py:69-70``.
    """
