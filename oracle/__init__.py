"""CPU oracle of the NanoKV sparse layer-step: test and baseline infrastructure only."""
