# Builds tests/_build/seam_check: the reference-side adapters
# (rapidllm_amd/integration/hip_engine.cpp, hip_device.cpp) compiled against the
# reference's own headers, with a driver that checks them on the GPU against the
# oracle.  Needs a RapidLLM tree for the headers (REF, default /root/reference);
# only headers are used, no reference source file is compiled.
#   make -f tests/seam_check.mk [REF=/path/to/RapidLLM]
ROOT := $(abspath $(dir $(lastword $(MAKEFILE_LIST)))/..)
REF ?= /root/reference
OUT := $(ROOT)/tests/_build/seam_check
SRCS := $(ROOT)/tests/seam_check.cpp $(ROOT)/rapidllm_amd/integration/hip_engine.cpp \
        $(ROOT)/rapidllm_amd/integration/hip_device.cpp
HDRS := $(ROOT)/rapidllm_amd/integration/hip_backend.h $(ROOT)/include/rapidllm_hip.h $(ROOT)/include/rl_model.h

$(OUT): $(SRCS) $(HDRS) $(ROOT)/rapidllm_amd/_lib/librapidllm_hip.so $(ROOT)/oracle/_build/liboracle.so
	mkdir -p $(dir $(OUT))
	g++ -std=c++20 -O2 -Wall -I$(REF)/include -I$(ROOT)/include -o $@ $(SRCS) \
	    -L$(ROOT)/rapidllm_amd/_lib -lrapidllm_hip -L$(ROOT)/oracle/_build -loracle \
	    -Wl,-rpath,'$$ORIGIN/../../rapidllm_amd/_lib:$$ORIGIN/../../oracle/_build'
