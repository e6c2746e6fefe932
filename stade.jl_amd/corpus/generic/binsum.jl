# binsum(loss, v, bins, c, i_n, i_b)
#
# A binned sum of squares: c[bins[i]] += v[i]^2 for every sample i (bins: Int64 labels in
# 1..i_b, many samples per bin), then loss += sum(c .^ 2).  The primal and its tangent
# accumulate into the small array c from every iteration.
#
# loss: length-1 output, accumulated; v: length i_n; bins: Int64 labels, length i_n;
# c: length i_b, accumulated; i_n: samples; i_b: bins
function binsum(loss, v, bins, c, i_n, i_b)
    for i = 1:i_n
        c[bins[i]] = c[bins[i]] + v[i] ^ 2
    end
    for b = 1:i_b
        loss[1] = loss[1] + c[b] ^ 2
    end
    return nothing
end
