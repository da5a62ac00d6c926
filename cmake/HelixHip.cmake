# HelixHip.cmake -- device code for gfx950 through hipcc.
#
# Counterpart of the reference's cmake/HelixMetal.cmake (which compiles the
# Metal kernels into a metallib): here the kernels become one code object
# (hipcc --genco) that the runtime loads with hipModuleLoadData, and the few
# translation units that hold device globals become ordinary objects
# (hipcc -c) linked into the library.
#
# Every device compile disables packed FP32 instructions
# (-target-feature -packed-fp32-ops) and keeps MFMA accumulators in VGPRs
# (-amdgpu-mfma-vgpr-form), the flags helix_amd/csrc/Makefile uses.

set(HELIX_ARCH "gfx950" CACHE STRING "AMDGPU target of the device code")
set(HELIX_ROCM "/opt/rocm" CACHE PATH "ROCm installation")
find_program(HELIX_HIPCC hipcc HINTS "${HELIX_ROCM}/bin" REQUIRED)

set(HELIX_HIP_DEVICE_FLAGS
    --offload-arch=${HELIX_ARCH} -O3 -std=c++17
    -Xclang -target-feature -Xclang -packed-fp32-ops)

# helix_hip_code_object(<target> <out.hsaco> <source.hip> DEPENDS <files...>)
#   Builds <out.hsaco>, a gfx950 code object with every kernel of <source.hip>.
function(helix_hip_code_object TARGET_NAME OUT SRC)
    cmake_parse_arguments(ARG "" "" "DEPENDS;INCLUDES" ${ARGN})
    set(incs "")
    foreach(d IN LISTS ARG_INCLUDES)
        list(APPEND incs "-I${d}")
    endforeach()
    add_custom_command(
        OUTPUT "${OUT}"
        COMMAND "${HELIX_HIPCC}" ${HELIX_HIP_DEVICE_FLAGS} --genco --no-gpu-bundle-output
                -mllvm -amdgpu-mfma-vgpr-form ${incs} "${SRC}" -o "${OUT}"
        DEPENDS "${SRC}" ${ARG_DEPENDS}
        COMMENT "hipcc --genco ${HELIX_ARCH}: ${SRC}"
        VERBATIM)
    add_custom_target(${TARGET_NAME} DEPENDS "${OUT}")
endfunction()

# helix_hip_object(<out.o> <source.hip> INCLUDES <dirs...> DEPENDS <files...>)
#   Host + device object of one HIP translation unit (its device globals are
#   registered with the HIP runtime when the program that links it starts).
function(helix_hip_object OUT SRC)
    cmake_parse_arguments(ARG "" "" "DEPENDS;INCLUDES" ${ARGN})
    set(incs "")
    foreach(d IN LISTS ARG_INCLUDES)
        list(APPEND incs "-I${d}")
    endforeach()
    add_custom_command(
        OUTPUT "${OUT}"
        COMMAND "${HELIX_HIPCC}" --offload-arch=${HELIX_ARCH} -O2 -fPIC -std=c++17 -c
                -Xclang -target-feature -Xclang -packed-fp32-ops ${incs} "${SRC}" -o "${OUT}"
        DEPENDS "${SRC}" ${ARG_DEPENDS}
        COMMENT "hipcc -c ${HELIX_ARCH}: ${SRC}"
        VERBATIM)
endfunction()
