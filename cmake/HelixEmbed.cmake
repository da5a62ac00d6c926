# HelixEmbed.cmake -- turn the code object into a C array so it ships inside
# libhelix.a (counterpart of the reference's cmake/HelixEmbed.cmake, which does
# the same for its metallibs): the library then carries no path into the build
# tree, and helix_ctx_create loads the embedded bytes with hipModuleLoadData.
#
# The array is generated at build time, so it tracks the code object.

# Captured at include time: inside the function CMAKE_CURRENT_LIST_DIR would
# name the caller's directory.
set(HELIX_EMBED_SCRIPT "${CMAKE_CURRENT_LIST_DIR}/HelixEmbedRun.cmake")

# helix_embed_code_object(<target> <in.hsaco> <symbol> <out.c> [DEPENDS <targets...>])
function(helix_embed_code_object TARGET_NAME IN SYMBOL OUT)
    cmake_parse_arguments(ARG "" "" "DEPENDS" ${ARGN})
    add_custom_command(
        OUTPUT "${OUT}"
        COMMAND ${CMAKE_COMMAND} -DHELIX_EMBED_IN=${IN} -DHELIX_EMBED_OUT=${OUT}
                -DHELIX_EMBED_SYM=${SYMBOL} -P "${HELIX_EMBED_SCRIPT}"
        DEPENDS "${IN}" "${HELIX_EMBED_SCRIPT}" ${ARG_DEPENDS}
        COMMENT "Embedding ${IN} as ${SYMBOL}"
        VERBATIM)
    add_custom_target(${TARGET_NAME} DEPENDS "${OUT}")
endfunction()
