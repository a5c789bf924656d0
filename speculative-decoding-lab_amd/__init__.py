"""MI355X (gfx950) paged-KV speculative-verify path.

Put this directory on ``sys.path`` and import ``engine`` / ``specdec``: the same
module names and signatures as the reference's ``engine/`` and ``specdec/``
packages, backed by the HIP library built from ``csrc/`` into ``lib/``.
"""
