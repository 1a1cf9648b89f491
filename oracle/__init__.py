"""CPU restatement of the reference path (test infrastructure; see lb_oracle.h)."""
