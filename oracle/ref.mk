# oracle/_ref: the parts of the reference that compile from their own sources
# here, built where they lie under the reference checkout (never copied).
# Only sources/scalar_math.h does: every other file of the path needs ggml's
# headers, which the checkout does not hold (its submodule is empty).
#
#   make -C oracle -f ref.mk REFERENCE=/root/reference
#
# clang++ as the reference's own build uses (C++20 for <bit>'s bit_cast); the
# header's expressions hold no multiplication an addition could contract.
REFERENCE ?= /root/reference
CXX := /opt/rocm/llvm/bin/clang++
OUT := _ref
LIB := $(OUT)/libref_scalar_math.so

all: $(LIB)

$(LIB): ref_scalar_math.cc $(REFERENCE)/sources/scalar_math.h
	@mkdir -p $(OUT)
	$(CXX) -std=c++20 -O2 -fPIC -shared -I$(REFERENCE)/sources ref_scalar_math.cc -o $@

clean:
	rm -rf $(OUT)

.PHONY: all clean
