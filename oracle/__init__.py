"""CPU restatement of the reference math — test infrastructure only."""
