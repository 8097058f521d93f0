"""Python callers of the MiniMind gfx950 runtime (import path of the
reference's src/python/minimind_orangepi package)."""
