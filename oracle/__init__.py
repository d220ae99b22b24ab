"""CPU oracle of the int8 linear path: test infrastructure only (see nx_oracle.cpp)."""
