function initstacks_flatmv_b()
    return nothing
end

function flatmv_b(loss, lossb, a, ab, x, xb, y, yb, i_m, i_n)
    for idx = 1:i_m * i_n
        i = div(idx - 1, i_n) + 1
        j = mod(idx - 1, i_n) + 1
        y[i] = y[i] + a[idx] * x[j]
    end
    for k = 1:i_m
        loss[1] = loss[1] + y[k] ^ 2
    end
    for k = i_m:-1:1
        yb[k] = yb[k] + 2 * y[k] * lossb[1]
    end
    for idx = i_m * i_n:-1:1
        i = div(idx - 1, i_n) + 1
        j = mod(idx - 1, i_n) + 1
        __cse_0 = yb[i]
        ab[idx] = ab[idx] + x[j] * __cse_0
        xb[j] = xb[j] + a[idx] * __cse_0
    end
    return nothing
end

function flatmv(loss, a, x, y, i_m, i_n)
    for idx = 1:i_m * i_n
        i = div(idx - 1, i_n) + 1
        j = mod(idx - 1, i_n) + 1
        y[i] = y[i] + a[idx] * x[j]
    end
    for k = 1:i_m
        loss[1] = loss[1] + y[k] ^ 2
    end
    return nothing
end
