"""`python -m axon <kernel-path> --sizes ...` runs the command-line driver."""

from enzyme_amd.cli import main

main()
