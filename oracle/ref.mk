# Compiles the reference engine's own C sources, where they lie under $(REF),
# together with ref_harness.c into oracle/_ref/libndref.so, and with the
# engine-side binding of the package's host library into
# oracle/_ref/libndrefgpu.so. Test
# infrastructure only: used to pin the oracle and as the "reference" CPU
# baseline. Output goes to _ref/ only; nothing from $(REF) is copied.
REF ?= /root/reference
CC ?= gcc
ENG = $(REF)/engine
CFLAGS = -std=gnu99 -O2 -fPIC -ffp-contract=off -w -I$(ENG)/include -I$(ENG)/src
SRCS = $(ENG)/src/nd_quant.c $(ENG)/src/nd_cact.c $(ENG)/src/nd_tokenizer.c

PKG = ../esp32-needle-3_amd

all: _ref/libndref.so _ref/libndrefgpu.so

_ref/libndref.so: ref_harness.c $(SRCS) $(ENG)/src/nd_model.c
	mkdir -p _ref
	$(CC) $(CFLAGS) -shared -o $@ ref_harness.c $(SRCS) -lm -lpthread

# The engine-side binding of libndhost (ref_engine_gpu.c), compiled against
# the engine's own nd_model.h / nd_model.c and linked against the package's
# libndhost.so and libndattn.so (found beside this tree at run time). Needs
# the package built first.
_ref/libndrefgpu.so: ref_engine_gpu.c ref_harness.c $(SRCS) $(ENG)/src/nd_model.c $(PKG)/libndhost.so
	mkdir -p _ref
	$(CC) $(CFLAGS) -I../include -shared -o $@ ref_engine_gpu.c $(SRCS) -L$(PKG) -lndhost -lndattn \
		-Wl,-rpath,'$$ORIGIN/../../esp32-needle-3_amd' -lm -lpthread

.PHONY: all _ref/libndref.so _ref/libndrefgpu.so
