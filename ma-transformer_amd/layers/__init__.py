"""Drop-in layer API of the reference's src/layers package."""
