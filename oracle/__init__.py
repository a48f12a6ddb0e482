"""C oracle of the reference arithmetic (test infrastructure only)."""
