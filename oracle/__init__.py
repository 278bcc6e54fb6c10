"""CPU oracle of the whisper.rs attention path: test infrastructure only."""
