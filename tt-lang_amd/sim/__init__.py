"""Drop-in for the `sim` helpers tt-lang examples import (sim.testing,
sim.typedefs)."""
