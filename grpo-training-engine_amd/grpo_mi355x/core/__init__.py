"""Mirror of the reference's ``src/core`` pieces on the rollout path."""
