# Compiles the reference's own CPU backend, src/dabsn/kernels/cpu_runtime.cpp, straight
# from /root/reference into oracle/_ref/ (TEST INFRASTRUCTURE ONLY: the tests use it to pin
# the C restatement in dabsn_oracle.c; nothing in the product loads it).
#
# This is not the reference's build system (cpu.py JIT-loads the file through
# torch.utils.cpp_extension.load): it is one g++ line over that one source file, with the
# flags the reference passes (-O3 -std=c++17 -ffp-contract=off -fopenmp, cpu.py:78,95-96)
# against the torch headers and libraries installed with the image's PyTorch.
#
#   make -f oracle/ref.mk            # builds oracle/_ref/dabsn_ref_cpu<EXT_SUFFIX>
#
# The module exposes the reference's pybind11 functions (cpu_runtime.cpp:1238-1261).
HERE := $(dir $(abspath $(lastword $(MAKEFILE_LIST))))
REF_SRC ?= /root/reference/src/dabsn/kernels/cpu_runtime.cpp
OUT := $(HERE)_ref
PY ?= python3
TORCH_DIR := $(shell $(PY) -c "import os, torch; print(os.path.dirname(torch.__file__))")
PY_INC := $(shell $(PY) -c "import sysconfig; print(sysconfig.get_paths()['include'])")
EXT := $(shell $(PY) -c "import sysconfig; print(sysconfig.get_config_var('EXT_SUFFIX'))")
ABI := $(shell $(PY) -c "import torch; print(int(torch._C._GLIBCXX_USE_CXX11_ABI))")
TARGET := $(OUT)/dabsn_ref_cpu$(EXT)

CXXFLAGS := -O3 -std=c++17 -ffp-contract=off -fopenmp -fPIC -shared -w \
  -DTORCH_EXTENSION_NAME=dabsn_ref_cpu -DTORCH_API_INCLUDE_EXTENSION_H \
  -D_GLIBCXX_USE_CXX11_ABI=$(ABI) \
  -isystem $(TORCH_DIR)/include -isystem $(TORCH_DIR)/include/torch/csrc/api/include \
  -isystem $(PY_INC)
LDFLAGS := -L$(TORCH_DIR)/lib -Wl,-rpath,$(TORCH_DIR)/lib -lc10 -ltorch -ltorch_cpu -ltorch_python

all: $(TARGET)

$(TARGET): $(REF_SRC) $(lastword $(MAKEFILE_LIST))
	@mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -o $@.tmp $(REF_SRC) $(LDFLAGS)
	mv $@.tmp $@

clean:
	rm -rf $(OUT)

.PHONY: all clean
