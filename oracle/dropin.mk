# Builds oracle/_ref/libhkbs_dropin.so: the C++ drop-in of this library
# (hikoboshi_amd/dropin/inverse_fold_hip.cpp) compiled against the reference's
# own, unmodified public headers, plus the test shim tests/csrc/dropin_check.cpp,
# linked to hikoboshi_amd/libhkbs_pmpnn.so. The reference headers it uses are
# header-only, so no reference object is linked. Test infrastructure; outputs go
# to oracle/_ref/ only.
#
#   make -f oracle/dropin.mk REF=/root/reference

REF ?= /root/reference
HERE := $(patsubst %/,%,$(dir $(lastword $(MAKEFILE_LIST))))
ROOT := $(HERE)/..
OUT := $(HERE)/_ref
CXX ?= g++
CXXFLAGS := -std=c++17 -O2 -fPIC -Wall -Wextra -I$(REF)/cpp/include -I$(ROOT)/include -I$(ROOT)/hikoboshi_amd/dropin
SRCS := $(ROOT)/hikoboshi_amd/dropin/inverse_fold_hip.cpp $(ROOT)/tests/csrc/dropin_check.cpp
LIB := $(ROOT)/hikoboshi_amd/libhkbs_pmpnn.so

all: $(OUT)/libhkbs_dropin.so

$(OUT)/libhkbs_dropin.so: $(SRCS) $(ROOT)/hikoboshi_amd/dropin/inverse_fold_hip.hpp $(ROOT)/include/hkbs_pmpnn.h $(LIB)
	@mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -shared -o $@ $(SRCS) -L$(ROOT)/hikoboshi_amd -lhkbs_pmpnn \
	  -Wl,-rpath,'$$ORIGIN/../../hikoboshi_amd' -Wl,--no-undefined

clean:
	rm -f $(OUT)/libhkbs_dropin.so

.PHONY: all clean
