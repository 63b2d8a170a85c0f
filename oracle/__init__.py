"""CPU oracle of the search path — test infrastructure only (see oracle/va_oracle.h)."""
