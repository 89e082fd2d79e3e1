# Builds oracle/_ref/libhkbs_ref.so from the reference's own, unmodified
# sources, read where they lie under the reference checkout, plus
# oracle/ref_driver.cpp. Test infrastructure only (the CPU checker and the
# CPU baseline). Outputs go to oracle/_ref/ only.
#
#   make -f oracle/ref.mk REF=/root/reference
#
# Flags: C++17, -O3, portable x86-64 target, no FMA contraction, and the
# reference's default "fast" GEMM parity mode (meson.options:118-124,
# meson.build:142-147).

REF ?= /root/reference
HERE := $(patsubst %/,%,$(dir $(lastword $(MAKEFILE_LIST))))
OUT := $(HERE)/_ref
CXX ?= g++
CXXFLAGS := -std=c++17 -O3 -fPIC -ffp-contract=off -DHIKOBOSHI_GEMM_PARITY_MODE_DEFAULT_FAST=1 \
            -I$(REF)/cpp/include -w

SRCS := \
  $(REF)/cpp/primitives/compute/atom_pair_distance_scalar.cpp \
  $(REF)/cpp/primitives/compute/axpy_scalar.cpp \
  $(REF)/cpp/primitives/compute/bias_add_scalar.cpp \
  $(REF)/cpp/primitives/compute/gelu_scalar.cpp \
  $(REF)/cpp/primitives/compute/knn_scalar.cpp \
  $(REF)/cpp/primitives/compute/rbf_scalar.cpp \
  $(REF)/cpp/primitives/compute/gather_scalar.cpp \
  $(REF)/cpp/primitives/compute/layer_norm_scalar.cpp \
  $(REF)/cpp/primitives/compute/log_softmax_scalar.cpp \
  $(REF)/cpp/primitives/compute/reduce_scalar.cpp \
  $(REF)/cpp/primitives/compute/softmax_scalar.cpp \
  $(REF)/cpp/primitives/linalg/gemm_scalar.cpp \
  $(REF)/cpp/primitives/linalg/gemm_scalar_fast.cpp \
  $(REF)/cpp/primitives/alignment/smith_waterman_scalar.cpp \
  $(REF)/cpp/primitives/alignment/soft_smith_waterman_scalar.cpp \
  $(REF)/cpp/primitives/alignment/traceback_scalar.cpp \
  $(REF)/cpp/dispatch/scalar_forward.cpp \
  $(REF)/cpp/modules/mpnn/edge_rbf_features_scalar.cpp \
  $(REF)/cpp/modules/mpnn/proteinmpnn_encoder_scalar.cpp \
  $(REF)/cpp/modules/mpnn/decoder_layer_scalar.cpp \
  $(REF)/cpp/modules/mpnn/decode_order_scalar.cpp \
  $(REF)/cpp/modules/mpnn/sampler_scalar.cpp \
  $(REF)/cpp/modules/mpnn/inverse_fold_scalar.cpp \
  $(REF)/cpp/algorithms/inverse_fold.cpp \
  $(REF)/cpp/io/design_fasta_writer.cpp \
  $(REF)/cpp/io/pdb_parser.cpp \
  $(REF)/cpp/io/mmcif_parser.cpp \
  $(REF)/cpp/io/structure_normalize.cpp \
  $(REF)/cpp/io/structure_atoms.cpp \
  $(REF)/cpp/io/atom_inference.cpp \
  $(REF)/cpp/io/atom_inference_kabsch.cpp \
  $(REF)/cpp/io/virtual_cb.cpp \
  $(REF)/cpp/io/residue_table.cpp \
  $(REF)/cpp/io/structure_loader.cpp

OBJS := $(patsubst $(REF)/cpp/%.cpp,$(OUT)/obj/%.o,$(SRCS)) $(OUT)/obj/ref_driver.o

all: $(OUT)/libhkbs_ref.so

$(OUT)/obj/%.o: $(REF)/cpp/%.cpp
	@mkdir -p $(dir $@)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/obj/ref_driver.o: $(HERE)/ref_driver.cpp
	@mkdir -p $(dir $@)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/libhkbs_ref.so: $(OBJS)
	$(CXX) -shared -o $@ $(OBJS) -Wl,--no-undefined -lm

clean:
	rm -rf $(OUT)

.PHONY: all clean
