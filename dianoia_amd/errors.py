"""The reference's Dart error types, as Python exceptions.

``ArgumentError`` is raised for bad arguments (unknown matrix, short lists,
invalid block data) and ``StateError`` for use after dispose or a failed GPU
command buffer, where the reference's Dart throws the errors of those names
(gpu.dart:1264-1267, 1327-1357; native.dart:633-641, 717-721).
``FormatException`` is raised for a weight cache that cannot be trusted
(q8_cache.dart:63-104).
"""


class ArgumentError(ValueError):
    pass


class StateError(RuntimeError):
    pass


class FormatException(ValueError):
    pass
