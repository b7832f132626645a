"""CPU oracle of the TAGI step -- test infrastructure, never imported by the engine."""
