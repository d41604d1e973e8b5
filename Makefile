# Per-case targets over eval/sizes.json, as in the reference's Makefile:39-46.
#
#   make rmsnorm_h4096        bench one case -> out/rmsnorm_h4096.csv (+ winners/)
#   make all / lnc1 / lnc2    every case / the single-device ones / the sharded ones
#   make rmsnorm              lists rmsnorm's case targets and exits 2
#   make clean-rmsnorm        removes every per-case artefact of rmsnorm
#   make lib                  (re)builds enzyme_amd/lib/libaxon_hip.so for gfx950
#   make test / test-gpu      CPU suite / GPU suite (pytest -m gpu)
#
# eval/gen_size_targets.py writes out/size_targets.mk, one file target
# out/<kernel>_<case>.csv per case, each depending on its spec package,
# eval/sizes.json and the HIP library. AXON_ARGS is passed to every run
# (e.g. AXON_ARGS="--candidate-budget 16 --bench 200").

PYTHON ?= python3
AXON_ARGS ?=
AXON_LIB := enzyme_amd/lib/libaxon_hip.so
AXON_SRCS := $(wildcard enzyme_amd/csrc/*.hip enzyme_amd/csrc/*.hpp include/*.h) enzyme_amd/build.py

KERNELS := $(patsubst kernels/%.py,%,$(wildcard kernels/*.py)) \
           $(patsubst kernels/%/__init__.py,%,$(wildcard kernels/*/__init__.py))

.DELETE_ON_ERROR:
.PHONY: all lnc1 lnc2 lib test test-gpu clean $(KERNELS) $(addprefix clean-,$(KERNELS))

all: $(CASE_TARGETS)

out/size_targets.mk: eval/sizes.json eval/gen_size_targets.py
	@mkdir -p out
	$(PYTHON) eval/gen_size_targets.py > $@

-include out/size_targets.mk

lnc1: $(LNC1_TARGETS)

lnc2: $(LNC2_TARGETS)

$(AXON_LIB): $(AXON_SRCS)
	$(PYTHON) -m enzyme_amd.build --incremental

lib:
	$(PYTHON) -m enzyme_amd.build

test:
	$(PYTHON) -m pytest tests -q -m "not gpu"

test-gpu:
	$(PYTHON) -u -m pytest tests -q -m gpu -x --timeout 120 --timeout-method thread

# A bare kernel name is ambiguous (a kernel has several cases): list them.
$(KERNELS): %:
	@echo "Pick a case for '$*'. Available case targets:"
	@for c in $(CASES_$*); do echo "  make $$c"; done
	@exit 2

$(addprefix clean-,$(KERNELS)): clean-%:
	@for c in $(CASES_$*); do \
		rm -f "out/$$c.csv"; \
		rm -rf "out/$$c/" "out/baseline_$$c/" "out/baseline_$$c.csv"; \
		rm -f "out/winners/$$c.py" "out/winners/$${c}_case.py"; \
	done

clean: $(addprefix clean-,$(KERNELS))
	rm -f out/size_targets.mk
