# The reference's own test programs, compiled from their sources where they
# lie (REF/tests/unit, REF/tests/integration) against this repository's
# headers and libraries: the check that code written against the reference's
# API builds and runs on this library with only the CUDA-runtime spellings
# changed (cuda_to_hip.sed).  Each source is piped through sed into the
# compiler; the only files written are the executables in _ref/.
#
#   make -f reference_programs.mk            (from oracle/; REF=/root/reference)
#
# The library must be built first (libqwen3_runtime.so, libq3k.so).  The
# executables find it through a relative rpath, so the tree can move.
REF ?= /root/reference
REPO := $(abspath $(CURDIR)/..)
LIB := $(REPO)/qwen3-runtime-byyourself_amd/lib
ROCM ?= /opt/rocm
OUT := _ref
CXX := g++
FLAGS := -O2 -std=c++17 -D__HIP_PLATFORM_AMD__ -I$(REPO)/include -I$(ROCM)/include
LIBS := -L$(LIB) -lqwen3_runtime -lq3k -L$(ROCM)/lib -lamdhip64 -pthread \
        -Wl,-rpath,'$$ORIGIN/../../qwen3-runtime-byyourself_amd/lib' -Wl,-rpath,$(ROCM)/lib

# Every unit test of a component this library provides, and the two
# integration programs that need only a safetensors file.  Not built: the
# GEMM tests (linear, lm_head), the tokenizer and chat template, and the
# programs that need a real checkpoint.
CPU_UNIT := core_metadata_test tensor_view_test tensor_cpu_test buffer_cpu_test model_config_test \
            mapped_file_test safetensors_file_test safetensors_checkpoint_test
GPU_UNIT := buffer_cuda_test tensor_cuda_test embedding_cuda_test rms_norm_cuda_test rope_cuda_test \
            elementwise_cuda_test kv_cache_cuda_test gqa_attention_cuda_test argmax_cuda_test sampler_cuda_test
INTEGRATION := safetensors_metadata_smoke safetensors_loader_smoke

all: $(addprefix $(OUT)/,$(CPU_UNIT) $(GPU_UNIT) $(INTEGRATION))

$(OUT):
	mkdir -p $@

$(OUT)/%: $(REF)/tests/unit/%.cpp cuda_to_hip.sed $(LIB)/libqwen3_runtime.so | $(OUT)
	sed -f cuda_to_hip.sed $< | $(CXX) $(FLAGS) -x c++ - -o $@ $(LIBS)

$(OUT)/%: $(REF)/tests/integration/%.cpp cuda_to_hip.sed $(LIB)/libqwen3_runtime.so | $(OUT)
	sed -f cuda_to_hip.sed $< | $(CXX) $(FLAGS) -x c++ - -o $@ $(LIBS)

clean:
	rm -rf $(OUT)

.PHONY: all clean
