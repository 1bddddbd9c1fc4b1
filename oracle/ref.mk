# TEST INFRASTRUCTURE ONLY: the reference's own CPU path (src/cpu/q8.c, src/cpu/expert.c, src/model/qtype.c),
# compiled from /root/reference where the sources lie (nothing copied), linked with this directory's driver
# (ref_driver.cc: C entry points over them) into oracle/_ref/libref.so. flags as the reference's Makefile:79-82 gives
# src/cpu (-ffp-contract=off -mavx2 -mfma -mf16c). q8.c is compiled as C++: ROCm's clang rejects its one non-constant
# rounding argument (q8.c:420, a `const int`) in C, and accepts it as the constant expression C++ makes of it; the
# code is the same.
REF ?= /root/reference
CLANG ?= /opt/rocm/lib/llvm/bin/clang
OUT := _ref
FLAGS := -O2 -fPIC -ffp-contract=off -mavx2 -mfma -mf16c -I$(REF)/include -I$(REF)/kernels

all: $(OUT)/libref.so

$(OUT)/q8.o: $(REF)/src/cpu/q8.c
	@mkdir -p $(OUT)
	$(CLANG) -x c++ -std=c++17 $(FLAGS) -c $< -o $@

$(OUT)/expert.o: $(REF)/src/cpu/expert.c
	@mkdir -p $(OUT)
	$(CLANG) -std=gnu11 $(FLAGS) -c $< -o $@

$(OUT)/qtype.o: $(REF)/src/model/qtype.c
	@mkdir -p $(OUT)
	$(CLANG) -std=gnu11 $(FLAGS) -c $< -o $@

$(OUT)/ref_driver.o: ref_driver.cc
	@mkdir -p $(OUT)
	$(CLANG) -x c++ -std=c++17 $(FLAGS) -c $< -o $@

$(OUT)/libref.so: $(OUT)/q8.o $(OUT)/expert.o $(OUT)/qtype.o $(OUT)/ref_driver.o
	$(CLANG) -shared -o $@ $^ -lm -lpthread -lstdc++

.PHONY: all
