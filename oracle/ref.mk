# Builds the reference's own CPU kernels (knn.cpp, fps.cpp) from where they
# lie under the reference checkout, into oracle/_ref/ (never committed).
# TEST INFRASTRUCTURE ONLY: tests/test_ref_cpu_kernels.py loads them in a
# separate process (they register the same torch.library namespaces as the
# product) to pin the oracle's tpo_cpu_* restatement and the product's CPU
# dispatch keys against the reference's code.
# Flags as the reference's setup.py:78-81 gives them: -O3 -std=c++17, no -march.
#   make -f ref.mk REF=/root/reference
REF ?= /root/reference
PY ?= python3
TORCH_INC := $(shell $(PY) -c "from torch.utils import cpp_extension as c; print(' '.join('-I' + p for p in c.include_paths()))")
TORCH_LIB := $(shell $(PY) -c "from torch.utils import cpp_extension as c; print(c.library_paths()[0])")
PY_INC := $(shell $(PY) -c "import sysconfig; print(sysconfig.get_paths()['include'])")
ABI := $(shell $(PY) -c "import torch; print(int(torch._C._GLIBCXX_USE_CXX11_ABI))")
CXXFLAGS = -O3 -std=c++17 -fPIC -shared -D_GLIBCXX_USE_CXX11_ABI=$(ABI) $(TORCH_INC) -I$(PY_INC)
LDFLAGS = -L$(TORCH_LIB) -Wl,-rpath,$(TORCH_LIB) -ltorch -ltorch_cpu -lc10
HERE := $(dir $(abspath $(lastword $(MAKEFILE_LIST))))
OUT := $(HERE)_ref

all: $(OUT)/knn_ref.so $(OUT)/fps_ref.so

$(OUT)/knn_ref.so: $(REF)/torch_point_ops/knn/csrc/knn.cpp
	mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -o $@ $< $(LDFLAGS)

$(OUT)/fps_ref.so: $(REF)/torch_point_ops/fps/csrc/fps.cpp
	mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -o $@ $< $(LDFLAGS)

.PHONY: all
