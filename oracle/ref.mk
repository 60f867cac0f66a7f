# Compiles the reference engine's own C sources, where they lie under $(REF),
# together with ref_harness.c into oracle/_ref/libndref.so. Test
# infrastructure only: used to pin the oracle and as the "reference" CPU
# baseline. Output goes to _ref/ only; nothing from $(REF) is copied.
REF ?= /root/reference
CC ?= gcc
ENG = $(REF)/engine
CFLAGS = -std=gnu99 -O2 -fPIC -ffp-contract=off -w -I$(ENG)/include -I$(ENG)/src
SRCS = $(ENG)/src/nd_quant.c $(ENG)/src/nd_cact.c $(ENG)/src/nd_tokenizer.c

_ref/libndref.so: ref_harness.c $(SRCS) $(ENG)/src/nd_model.c
	mkdir -p _ref
	$(CC) $(CFLAGS) -shared -o $@ ref_harness.c $(SRCS) -lm -lpthread

.PHONY: _ref/libndref.so
