# Builds programs from the reference's own C++ sources into _ref/ (kept out of
# the repository).  Only header-only code that compiles with the system
# compiler is used: hls/common/test_memh.hpp (the memh readers of the HLS
# testbenches), driven by memh_reader.cpp.
REF     ?= /root/reference
CXX     ?= g++
OUT     := _ref

all: $(OUT)/memh_reader

$(OUT)/memh_reader: memh_reader.cpp $(REF)/hls/common/test_memh.hpp
	mkdir -p $(OUT)
	$(CXX) -O2 -std=c++17 -Wall -I$(REF)/hls/common -o $@ memh_reader.cpp

clean:
	rm -rf $(OUT)

.PHONY: all clean
